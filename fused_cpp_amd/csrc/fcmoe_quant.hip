// fcmoe_quant.hip -- row quantisation, weight quantisation/packing and the
// BF16 activation pass.
//
// Row kernels: bf16 activation rows (cols % 8 == 0, up to 16384 columns) use
// one workgroup per row with the row held in registers; other rows use one
// wavefront per row (a strided max|x| pass, a butterfly, then the quantise
// pass). These are HBM-bound byte kernels (2 bytes in, 1 byte out per element).
#include "fcmoe_device.h"
#include "fcmoe_internal.h"
#include "fcmoe_quant_row.h"

namespace fcmoe {

namespace {

constexpr int kRowsPerBlock = 4;

__device__ __forceinline__ float load_x(const void* x, int x_is_f32, int64_t i) {
  return x_is_f32 ? ((const float*)x)[i] : bf16_to_f32(((const uint16_t*)x)[i]);
}

__global__ __launch_bounds__(kRowsPerBlock * kWave) void quant_rows_kernel(const void* x, int x_is_f32,
                                                                            int64_t rows, int64_t cols,
                                                                            int rounding, int8_t* q, int64_t ldq,
                                                                            float* scales) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  const int64_t base = row * cols;
  float m = 0.0f;
  if (!x_is_f32 && (cols % 8) == 0) {
    const uint4* p = (const uint4*)((const uint16_t*)x + base);
    for (int64_t i = lane; i < cols / 8; i += kWave) {
      uint4 v = p[i];
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        m = fmaxf(m, fabsf(__uint_as_float(w[j] << 16)));
        m = fmaxf(m, fabsf(__uint_as_float(w[j] & 0xffff0000u)));
      }
    }
  } else {
    for (int64_t i = lane; i < cols; i += kWave) m = fmaxf(m, fabsf(load_x(x, x_is_f32, base + i)));
  }
  m = wave_max(m);
  const float scale = m > 0.0f ? m / 127.0f : 1.0f;
  const float inv = 1.0f / scale;
  if (lane == 0) scales[row] = scale;
  int8_t* qr = q + row * ldq;
  if (!x_is_f32 && (cols % 8) == 0 && (ldq % 8) == 0) {
    const uint4* p = (const uint4*)((const uint16_t*)x + base);
    for (int64_t i = lane; i < cols / 8; i += kWave) {
      uint4 v = p[i];
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t a = (uint8_t)quant_value(__uint_as_float(w[j] << 16), scale, inv, rounding);
        const uint32_t b = (uint8_t)quant_value(__uint_as_float(w[j] & 0xffff0000u), scale, inv, rounding);
        const uint32_t pair = a | (b << 8);
        if (j < 2)
          lo |= pair << (16 * j);
        else
          hi |= pair << (16 * (j - 2));
      }
      ((uint2*)qr)[i] = make_uint2(lo, hi);
    }
  } else {
    for (int64_t i = lane; i < cols; i += kWave) qr[i] = quant_value(load_x(x, x_is_f32, base + i), scale, inv, rounding);
  }
  for (int64_t i = cols + lane; i < ldq; i += kWave) qr[i] = 0;
}

// bf16 rows with cols % 8 == 0 and ldq % 8 == 0 (every activation row of the
// MoE and i8gemm paths): one kRowThreads workgroup per row (quant_row_wg).
template <int CAP>
__global__ __launch_bounds__(kRowThreads) void quant_rows_wg_kernel(const uint16_t* x, int64_t cols, int rounding,
                                                                     int8_t* q, int64_t ldq, float* scales) {
  __shared__ float wmax[kRowThreads / kWave];
  quant_row_wg<CAP>(x, cols, rounding, q, ldq, scales, (int64_t)blockIdx.x, true, (int)threadIdx.x, wmax);
}

// W8A8 intermediate requant: y rows are bf16; the W13 epilogue left the max
// |y| of each 16-channel gate tile in rowpart, and the row scale uses their
// maximum. This is quantize_bf16_row applied to the intermediate
// (kernels.cpp:650-657).
__global__ __launch_bounds__(kRowsPerBlock * kWave) void requant_kernel(const uint16_t* y, int64_t ldy, int64_t rows,
                                                                         int64_t cols, const float* rowpart,
                                                                         int64_t parts, int8_t* q, int64_t ldq,
                                                                         float* scales) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  // max over the row's per-tile maxima (max is exact in any order)
  float m = 0.0f;
  for (int64_t i = lane; i < parts; i += kWave) m = fmaxf(m, rowpart[row * parts + i]);
  m = wave_max(m);
  const float scale = m > 0.0f ? m / 127.0f : 1.0f;
  const float inv = 1.0f / scale;
  if (lane == 0) scales[row] = scale;
  const uint4* p = (const uint4*)(y + row * ldy);
  uint2* qr = (uint2*)(q + row * ldq);
  // cols is a multiple of 16 and ldq of 64 (checked by the host).
  for (int64_t i = lane; i < ldq / 8; i += kWave) {
    uint32_t lo = 0, hi = 0;
    if (i * 8 < cols) {
      uint4 v = p[i];
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t a = (uint8_t)quant_value(__uint_as_float(w[j] << 16), scale, inv, 0);
        const uint32_t b = (uint8_t)quant_value(__uint_as_float(w[j] & 0xffff0000u), scale, inv, 0);
        const uint32_t pair = a | (b << 8);
        if (j < 2)
          lo |= pair << (16 * j);
        else
          hi |= pair << (16 * (j - 2));
      }
    }
    qr[i] = make_uint2(lo, hi);
  }
}

// Per-output-channel weight quantisation (kernels.cpp:451-457):
// scale = max|w|/127 (1 if 0), q = clamp(rint(w / scale), -127, 127).
__global__ __launch_bounds__(kRowsPerBlock * kWave) void quant_weight_kernel(const uint16_t* w, int64_t rows,
                                                                              int64_t cols, int8_t* q,
                                                                              float* scales) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  const uint16_t* src = w + row * cols;
  float m = 0.0f;
  for (int64_t i = lane; i < cols; i += kWave) m = fmaxf(m, fabsf(bf16_to_f32(src[i])));
  m = wave_max(m);
  const float scale = m > 0.0f ? m / 127.0f : 1.0f;
  if (lane == 0) scales[row] = scale;
  for (int64_t i = lane; i < cols; i += kWave) {
    float v = rintf(bf16_to_f32(src[i]) / scale);
    v = fmaxf(fminf(v, 127.0f), -127.0f);
    q[row * cols + i] = (int8_t)(int)v;
  }
}

// Pack [experts, n, k] (elem bytes eb) into 1 KiB tiles: for group g, channel
// tile t (16 channels), K chunk c (64 bytes): lane l holds channel
// g*n_half + t*16 + l%16, bytes c*64 + (l/16)*16 .. +16 of that channel's row.
// This is the operand order of v_mfma_i32_16x16x64_i8 / v_mfma_f32_16x16x32_bf16
// for the B matrix, so a wavefront streams one tile with one coalesced
// 16-byte load per lane. Padding (channels >= n_half, bytes >= k*eb) is zero.
__global__ __launch_bounds__(256) void pack_kernel(const uint8_t* src, int eb, int64_t n_half, int64_t k,
                                                    int n_groups, int64_t n_tiles, int64_t k_chunks,
                                                    int64_t expert_bytes, uint8_t* dst) {
  const int64_t expert = blockIdx.y;
  const int64_t per_expert_units = (int64_t)n_groups * n_tiles * k_chunks * kWave;  // 16-byte units
  const int64_t unit = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (unit >= per_expert_units) return;
  const int lane = (int)(unit % kWave);
  int64_t rest = unit / kWave;
  const int64_t c = rest % k_chunks;
  rest /= k_chunks;
  const int64_t t = rest % n_tiles;
  const int64_t g = rest / n_tiles;
  const int64_t ch_in_group = t * 16 + lane % 16;
  const int64_t row_bytes = k * eb;
  const int64_t byte0 = c * 64 + (lane / 16) * 16;
  uint8_t buf[16];
  const bool ch_ok = ch_in_group < n_half;
  const uint8_t* srow = src + (expert * (int64_t)n_groups * n_half + g * n_half + ch_in_group) * row_bytes;
#pragma unroll
  for (int j = 0; j < 16; ++j) buf[j] = (ch_ok && byte0 + j < row_bytes) ? srow[byte0 + j] : 0;
  uint4 v;
  v.x = buf[0] | (buf[1] << 8) | (buf[2] << 16) | ((uint32_t)buf[3] << 24);
  v.y = buf[4] | (buf[5] << 8) | (buf[6] << 16) | ((uint32_t)buf[7] << 24);
  v.z = buf[8] | (buf[9] << 8) | (buf[10] << 16) | ((uint32_t)buf[11] << 24);
  v.w = buf[12] | (buf[13] << 8) | (buf[14] << 16) | ((uint32_t)buf[15] << 24);
  ((uint4*)(dst + expert * expert_bytes))[unit] = v;
}

// BF16 interleaved activation pass (swigluoai: gate = column 2f, up = 2f+1;
// csrc/moe/arm/common/fused_moe_bf16_tiled.cpp:1894-1914). gate_up holds the
// W13 output in packed channel order: logical channel c < F at c, c >= F at
// fp16 + (c - F).
__global__ __launch_bounds__(256) void act_bf16_kernel(const float* gate_up, int64_t ldg, int64_t rows, int64_t f,
                                                        int64_t fp16, int mode, uint16_t* y, int64_t ldy) {
  const int64_t col = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (col >= ldy) return;
  for (int64_t row = blockIdx.y; row < rows; row += gridDim.y) {  // grid.y is capped at 65535
  if (col >= f) {
    y[row * ldy + col] = 0;
    continue;
  }
  const float* g = gate_up + row * ldg;
  auto at = [&](int64_t c) { return g[c < f ? c : fp16 + (c - f)]; };
  float v;
  if (mode == FCMOE_ACT_SWIGLUOAI) {
    const float gate = fminf(at(2 * col), 7.0f);
    const float up = fmaxf(-7.0f, fminf(at(2 * col + 1), 7.0f));
    const float glu = gate / (1.0f + expf(-gate * 1.702f));
    v = (up + 1.0f) * glu;
  } else {
    v = 0.0f;
  }
  y[row * ldy + col] = f32_to_bf16(v);
  }
}

__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

int fill_u32_launch(uint32_t* p, int64_t n, uint32_t v, hipStream_t stream) {
  if (n <= 0) return FCMOE_OK;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream, p, n, v);
  return check_launch("fill");
}

int quant_rows_launch(const void* x, int x_is_f32, int64_t rows, int64_t cols, int rounding, int8_t* q, int64_t ldq,
                      float* scales, hipStream_t stream) {
  if (rows <= 0) return FCMOE_OK;
  if (!x_is_f32 && cols % 8 == 0 && ldq % 8 == 0 && rows <= INT32_MAX) {
    const int64_t per_thread = ceil_div(cols / 8, kRowThreads);
    const dim3 grid((unsigned)rows), block(kRowThreads);
    const uint16_t* xb = (const uint16_t*)x;
    if (per_thread <= 1) {
      hipLaunchKernelGGL(quant_rows_wg_kernel<1>, grid, block, 0, stream, xb, cols, rounding, q, ldq, scales);
      return check_launch("quant_rows");
    }
    if (per_thread <= 2) {
      hipLaunchKernelGGL(quant_rows_wg_kernel<2>, grid, block, 0, stream, xb, cols, rounding, q, ldq, scales);
      return check_launch("quant_rows");
    }
    if (per_thread <= 4) {
      hipLaunchKernelGGL(quant_rows_wg_kernel<4>, grid, block, 0, stream, xb, cols, rounding, q, ldq, scales);
      return check_launch("quant_rows");
    }
    if (per_thread <= 8) {
      hipLaunchKernelGGL(quant_rows_wg_kernel<8>, grid, block, 0, stream, xb, cols, rounding, q, ldq, scales);
      return check_launch("quant_rows");
    }
  }
  hipLaunchKernelGGL(quant_rows_kernel, dim3((unsigned)ceil_div(rows, kRowsPerBlock)), dim3(kRowsPerBlock * kWave),
                     0, stream, x, x_is_f32, rows, cols, rounding, q, ldq, scales);
  return check_launch("quant_rows");
}

int requant_launch(const uint16_t* y, int64_t ldy, int64_t rows, int64_t cols, const float* rowpart, int64_t parts,
                   int8_t* q,
                   int64_t ldq, float* scales, hipStream_t stream) {
  if (rows <= 0) return FCMOE_OK;
  hipLaunchKernelGGL(requant_kernel, dim3((unsigned)ceil_div(rows, kRowsPerBlock)), dim3(kRowsPerBlock * kWave), 0,
                     stream, y, ldy, rows, cols, rowpart, parts, q, ldq, scales);
  return check_launch("requant");
}

int act_bf16_launch(const float* gate_up, int64_t ldg, int64_t rows, int64_t f, int64_t fp16, int mode, uint16_t* y,
                    int64_t ldy, hipStream_t stream) {
  if (rows <= 0) return FCMOE_OK;
  hipLaunchKernelGGL(act_bf16_kernel, dim3((unsigned)ceil_div(ldy, 256), (unsigned)(rows < 65535 ? rows : 65535)),
                     dim3(256), 0, stream,
                     gate_up, ldg, rows, f, fp16, mode, y, ldy);
  return check_launch("act_bf16");
}

}  // namespace fcmoe

using namespace fcmoe;

extern "C" int fcmoe_quantize_weight_rows(const uint16_t* w, int64_t rows, int64_t cols, int8_t* q, float* scales,
                                          hipStream_t stream) {
  if (rows < 0 || cols <= 0 || !w || !q || !scales) return fail(FCMOE_EINVAL, "quantize_weight_rows: bad args");
  if (rows == 0) return FCMOE_OK;
  hipLaunchKernelGGL(quant_weight_kernel, dim3((unsigned)ceil_div(rows, kRowsPerBlock)), dim3(kRowsPerBlock * kWave),
                     0, stream, w, rows, cols, q, scales);
  return check_launch("quantize_weight_rows");
}

extern "C" int64_t fcmoe_packed_expert_bytes(int elem_bytes, int64_t n, int64_t k, int n_groups) {
  if ((elem_bytes != 1 && elem_bytes != 2) || n <= 0 || k <= 0 || n_groups < 1 || n % n_groups) return -1;
  const int64_t n_half = n / n_groups;
  return (int64_t)n_groups * round_up(n_half, 16) * round_up(k * elem_bytes, 64);
}

extern "C" int fcmoe_pack_experts(const void* src, int elem_bytes, int64_t experts, int64_t n, int64_t k,
                                  int n_groups, void* dst, hipStream_t stream) {
  const int64_t eb = fcmoe_packed_expert_bytes(elem_bytes, n, k, n_groups);
  if (eb < 0 || experts < 0 || !src || !dst) return fail(FCMOE_EINVAL, "pack_experts: bad args");
  if (experts == 0) return FCMOE_OK;
  if (experts > 65535) return fail(FCMOE_EINVAL, "pack_experts: too many experts");
  const int64_t n_half = n / n_groups;
  const int64_t n_tiles = ceil_div(n_half, 16);
  const int64_t k_chunks = ceil_div(k * elem_bytes, 64);
  const int64_t units = (int64_t)n_groups * n_tiles * k_chunks * kWave;
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)ceil_div(units, 256), (unsigned)experts), dim3(256), 0, stream,
                     (const uint8_t*)src, elem_bytes, n_half, k, n_groups, n_tiles, k_chunks, eb, (uint8_t*)dst);
  return check_launch("pack_experts");
}

extern "C" int fcmoe_quantize_rows(const void* x, int x_is_f32, int64_t rows, int64_t cols, int rounding, int8_t* q,
                                   int64_t ldq, float* scales, hipStream_t stream) {
  if (rows < 0 || cols <= 0 || ldq < cols || (rounding != 0 && rounding != 1) || (x_is_f32 && rounding == 0))
    return fail(FCMOE_EINVAL, "quantize_rows: bad args");
  return quant_rows_launch(x, x_is_f32, rows, cols, rounding, q, ldq, scales, stream);
}
