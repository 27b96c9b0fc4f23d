// fcmoe_quant_row.h -- per-row activation quantisation shared by the row
// quantisation kernel (fcmoe_quant.hip) and the small-batch route kernel that
// also quantises the token rows (fcmoe_route.hip).
#pragma once

#include "fcmoe_device.h"

namespace fcmoe {

// rounding 0: quantize_bf16_row (csrc/moe/arm/i8mm_w8a8/kernels.cpp:211-228)
//   q = roundf(clamp(x * (1/s), -127, 127))  (half away from zero)
// rounding 1: i8gemm (csrc/i8gemm.cpp:368-392, tests/test_i8gemm.py:25-28)
//   q = clamp(rintf(x / s), -128, 127)       (ties to even)
__device__ __forceinline__ int8_t quant_value(float v, float scale, float inv, int rounding) {
  if (rounding == 0) {
    float t = v * inv;
    t = fmaxf(fminf(t, 127.0f), -127.0f);
    return (int8_t)(int)roundf(t);
  }
  float q = rintf(v / scale);
  q = fmaxf(fminf(q, 127.0f), -128.0f);
  return (int8_t)(int)q;
}

// Threads that quantise one bf16 row (cols % 8 == 0, ldq % 8 == 0).
constexpr int kRowThreads = 256;

// One bf16 row by kRowThreads threads (tid = 0 .. kRowThreads - 1): the row
// stays in registers (CAP 16-byte units per thread) between the max pass and
// the quantise pass, so it is read from HBM once and all its loads are in
// flight together. wmax: kRowThreads / kWave floats of LDS for this row.
// Contains one __syncthreads(): every thread of the workgroup calls it once;
// an inactive group (row past the end) loads and stores nothing.
template <int CAP>
__device__ __forceinline__ void quant_row_wg(const uint16_t* x, int64_t cols, int rounding, int8_t* q, int64_t ldq,
                                             float* scales, int64_t row, bool active, int tid, float* wmax) {
  const int64_t units = active ? cols / 8 : 0;
  const uint4* p = (const uint4*)(x + row * cols);
  uint4 v[CAP];
#pragma unroll
  for (int k = 0; k < CAP; ++k) {
    const int64_t i = tid + (int64_t)k * kRowThreads;
    v[k] = i < units ? p[i] : make_uint4(0, 0, 0, 0);  // zero units leave the max unchanged
  }
  float m = 0.0f;
#pragma unroll
  for (int k = 0; k < CAP; ++k) {
    const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m = fmaxf(m, fabsf(__uint_as_float(w[j] << 16)));
      m = fmaxf(m, fabsf(__uint_as_float(w[j] & 0xffff0000u)));
    }
  }
  m = wave_max(m);
  if (tid % kWave == 0) wmax[tid / kWave] = m;
  __syncthreads();
  if (!active) return;
#pragma unroll
  for (int w = 0; w < kRowThreads / kWave; ++w) m = fmaxf(m, wmax[w]);
  const float scale = m > 0.0f ? m / 127.0f : 1.0f;
  const float inv = 1.0f / scale;
  if (tid == 0) scales[row] = scale;
  int8_t* qr = q + row * ldq;
#pragma unroll
  for (int k = 0; k < CAP; ++k) {
    const int64_t i = tid + (int64_t)k * kRowThreads;
    if (i < units) {
      const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
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
  }
  for (int64_t i = cols + tid; i < ldq; i += kRowThreads) qr[i] = 0;
}

}  // namespace fcmoe
