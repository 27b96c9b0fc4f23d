// fcmoe_probe.hip -- measurement probes behind the figures the design quotes
// for this chip: the HBM streaming ceiling (loads to VGPRs and LDS-DMA), the
// MFMA + LDS-fragment loop rate by wave tile and waves per SIMD, a CU running
// MFMA waves and streaming waves side by side, and the cost of one agent-scope
// release per workgroup. Each entry enqueues one launch on `stream`; the
// caller times it (bench.py --probe). None of them is on the operators' path:
// this file builds into libfcmoe_probe.so (declared in fcmoe_probe.h), which
// only the benchmark loads, not into libfcmoe.so.
#include <stdint.h>

#include "fcmoe_device.h"
#include "fcmoe_internal.h"
#include "fcmoe_probe.h"

namespace fcmoe {
namespace {

typedef __attribute__((address_space(3))) void* probe_lds_ptr;

// Each wave streams `chunks` consecutive KiB of `src` (its own region) with an
// 8-deep ring of nontemporal 16-byte loads per lane (mode 0), or through
// buffer_load ... lds into its own 8 KiB ring of the dynamic LDS (mode 1). The
// dynamic LDS size (at least waves x 8 KiB in mode 1) also limits how many
// workgroups share a CU.
__global__ __launch_bounds__(1024) void probe_stream_kernel(const uint8_t* src, int64_t chunks, int mode, int* sink) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t dyn[];
  uint8_t* const ring_lds = dyn + (threadIdx.x / kWave) * 8192;
  const int lane = threadIdx.x % kWave;
  const int64_t gw = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  const uint8_t* base = src + gw * chunks * 1024;
  v4i acc = {0, 0, 0, 0};
  if (mode == 1) {
#if __HIP_DEVICE_COMPILE__
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, 0x7ffffff0, 0x00020000);
    for (int64_t c = 0; c < chunks; ++c) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (probe_lds_ptr)(ring_lds + (c % 8) * 1024), 16,
                                               lane * 16, (int)(c * 1024), 0, 2);
      if (c >= 7) __builtin_amdgcn_s_waitcnt((7 & 15) | (7 << 4) | (15 << 8));
    }
    __builtin_amdgcn_s_waitcnt(0);
#endif
    acc[0] = ring_lds[lane];
  } else {
    const v4i* p = (const v4i*)base + lane;
    v4i ring[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) ring[s] = __builtin_nontemporal_load(p + (s < chunks ? s : chunks - 1) * kWave);
    for (int64_t c = 0; c < chunks; c += 8) {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        acc += ring[s];
        int64_t n = c + s + 8;
        if (n >= chunks) n = chunks - 1;
        ring[s] = __builtin_nontemporal_load(p + n * kWave);
      }
    }
  }
  if (acc[0] == 0x7fffabcd) sink[0] = acc[1];  // keeps the loads; never true for the probe's data
}

// MFMA loop: per iteration a wave reads FM + FN fragments from LDS and issues
// FM * FN v_mfma_i32_16x16x64_i8 (the register reuse of an FM x FN wave tile).
template <int FM, int FN, int THREADS>
__global__ __launch_bounds__(THREADS) void probe_mfma_kernel(int iters, int* sink) {
  __shared__ v4i lds[64 * kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  for (int i = threadIdx.x; i < 64 * kWave; i += blockDim.x) lds[i] = v4i{i, 1, 2, 3};
  __syncthreads();
  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};
  for (int it = 0; it < iters; ++it) {
    v4i b[FN], a[FM];
#pragma unroll
    for (int j = 0; j < FN; ++j) b[j] = lds[((it + j * 7 + wave) & 63) * kWave + lane];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      a[i] = lds[((it * 3 + i * 5 + wave + 11) & 63) * kWave + lane];
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }
  v4i t = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) t += acc[i][j];
  if (t[0] == 0x7fffabcd) sink[threadIdx.x] = t[1];
}

// One workgroup per CU (LDS): waves [0, nc) run an MFMA + LDS-read loop (2
// fragment reads per 7 MFMAs), waves [nc, nc + ns) stream `chunks` KiB each
// from HBM (8-deep nontemporal ring, VALU accumulate, or MFMAs on the streamed
// data when stream_mfma).
__global__ __launch_bounds__(1024) void probe_mix_kernel(const uint8_t* src, int64_t chunks, int nc, int ns, int iters,
                                                         int stream_mfma, int* sink) {
  __shared__ v4i lds[96 * 1024 / 16];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  v4i acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = v4i{0, 0, 0, 0};
  if (wave < nc) {
    for (int i = lane; i < 96 * kWave; i += kWave) lds[i] = v4i{i, 1, 2, 3};
    const v4i a = lds[lane], b = lds[lane + kWave];
    for (int it = 0; it < iters; ++it) {
      const v4i x = lds[((it * 3 + wave) & 63) * kWave + lane];
      const v4i y = lds[((it * 5 + wave + 7) & 63) * kWave + lane];
#pragma unroll
      for (int j = 0; j < 7; ++j)
        acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(j & 1 ? x : a, j & 2 ? y : b, acc[j], 0, 0, 0);
    }
  } else if (wave < nc + ns) {
    const int64_t gw = (int64_t)blockIdx.x * ns + (wave - nc);
    const v4i* p = (const v4i*)(src + gw * chunks * 1024) + lane;
    v4i ring[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) ring[s] = __builtin_nontemporal_load(p + s * kWave);
    for (int64_t c = 0; c + 8 <= chunks; c += 8) {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        if (stream_mfma)
          acc[s & 3] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ring[s], ring[(s + 1) & 7], acc[s & 3], 0, 0, 0);
        else
          acc[0] += ring[s];
        int64_t n = c + s + 8;
        if (n >= chunks) n = chunks - 1;
        ring[s] = __builtin_nontemporal_load(p + n * kWave);
      }
    }
  }
  v4i t = acc[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) t += acc[i];
  if (t[0] == 0x7fffabcd) sink[threadIdx.x] = t[1];
}

// The streaming loop of probe_stream_kernel (mode 0), then, when `release`,
// each wave stores 1 KiB, makes it visible device-wide with an agent-scope
// release fence and bumps a counter; the 16th workgroup of each group of 16
// acquires and reads another wave's row (the last-arriver pattern).
__global__ __launch_bounds__(1024) void probe_fence_kernel(const uint8_t* src, int64_t chunks, int release, int* counters,
                                                           v4i* rows) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t gw = (int64_t)blockIdx.x * (blockDim.x / kWave) + wave;
  const v4i* p = (const v4i*)(src + gw * chunks * 1024) + lane;
  v4i acc = {0, 0, 0, 0};
  v4i ring[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) ring[s] = __builtin_nontemporal_load(p + (s < chunks ? s : chunks - 1) * kWave);
  for (int64_t c = 0; c < chunks; c += 8) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      acc += ring[s];
      int64_t n = c + s + 8;
      if (n >= chunks) n = chunks - 1;
      ring[s] = __builtin_nontemporal_load(p + n * kWave);
    }
  }
  if (!release) {
    if (acc[0] == 0x7fffabcd) rows[0] = acc;
    return;
  }
  rows[gw * kWave + lane] = acc;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  __shared__ int last;
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(counters + blockIdx.x / 16, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 15;
  __syncthreads();
  if (last) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    rows[gw * kWave + lane] = acc + rows[(gw ^ 1) * kWave + lane];
  }
}

// The prefill GEMM's load mix without its arithmetic: per K chunk every one
// of the 8 waves issues 4 one-KiB weight loads (a contiguous HBM stream per
// workgroup, nontemporal) and NA one-KiB loads of A rows (8 rows x 128
// bytes, 7168-byte row stride, from a 2 MiB window per XCD that stays in its
// L2), all by buffer_load ... lds into a 2-stage LDS ring. It keeps D chunks
// of loads in flight: wait for chunk c, meet at a barrier (BAR), issue chunk
// c + D.
template <int D, int NA, int BAR>
__global__ __launch_bounds__(512) void probe_ring_kernel(const uint8_t* src, const uint8_t* arows, int64_t chunks,
                                                         int* sink) {
#if __HIP_DEVICE_COMPILE__
  constexpr int NB = 4;
  constexpr int L = NB + NA;
  __shared__ __attribute__((aligned(1024))) uint8_t ring[2 * 8 * L * 1024];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(src + (int64_t)blockIdx.x * chunks * 8 * NB * 1024), (short)0, 0x7ffffff0, 0x00020000);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(arows + (int64_t)(blockIdx.x % 8) * (2 << 20)), (short)0, 2 << 20, 0x00020000);
  const uint32_t boff = (uint32_t)(wave * NB * 1024 + lane * 16);
  const uint32_t aoff = (uint32_t)((wave * NA * 8 + lane / 8) * 7168 + (lane % 8) * 16);
  auto issue = [&](int64_t c) {
    const int64_t cc = c < chunks ? c : chunks - 1;
    probe_lds_ptr dst = (probe_lds_ptr)(ring + ((c & 1) * 8 * L + wave * L) * 1024);
#pragma unroll
    for (int u = 0; u < NB; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (probe_lds_ptr)((uint8_t __attribute__((address_space(3)))*)dst + u * 1024),
                                               16, boff + u * 1024, (int)(cc * 8 * NB * 1024), 0, 2);
#pragma unroll
    for (int u = 0; u < NA; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (probe_lds_ptr)((uint8_t __attribute__((address_space(3)))*)dst + (NB + u) * 1024),
                                               16, aoff + u * 8 * 7168, (int)((cc % 56) * 128), 0, 0);
  };
#pragma unroll
  for (int c = 0; c < D; ++c) issue(c);
  for (int64_t c = 0; c < chunks; ++c) {
    constexpr int W = (D - 1) * L;
    __builtin_amdgcn_s_waitcnt((W & 15) | ((W >> 4) << 14) | (7 << 4) | (15 << 8));
    if (BAR) __builtin_amdgcn_s_barrier();
    issue(c + D);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (ring[lane] == 0x5a && lane == kWave) sink[0] = 1;  // never true: keeps the loads
#endif
}

template <int FM, int FN, int W>
int launch_mfma(int workgroups, int iters, int* sink, hipStream_t stream) {
  hipLaunchKernelGGL((probe_mfma_kernel<FM, FN, W * kWave>), dim3(workgroups), dim3(W * kWave), 0, stream, iters, sink);
  return check_launch("probe_mfma");
}


// The 256-row persistent tile's K loop (128 x 64 per wave, 8 waves) on LDS
// data, with optional per-iteration barrier and LDS-DMA traffic (see
// fcmoe_probe_loop_dma).
__global__ __launch_bounds__(512) void probe_loop_dma_kernel(const uint8_t* src, int mode, int iters, int* sink) {
#if __HIP_DEVICE_COMPILE__
  constexpr int FM = 8, FN = 4;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[96 * 1024 + 64 * 1024];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  for (int i = threadIdx.x; i < 96 * 1024 / 16; i += blockDim.x) ((v4i*)smem)[i] = v4i{i, 1, 2, 3};
  __syncthreads();
  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, 1 << 20, 0x00020000);
  const int base = __builtin_amdgcn_readfirstlane((int)(blockIdx.x % 8) * 65536);
  const uint8_t* sa = smem + (wave / 4) * 32768 + lane * 16;
  const uint8_t* sb = smem + 65536 + (wave % 4) * FN * 1024 + lane * 16;
  for (int it = 0; it < iters; ++it) {
    if (mode & 4) __builtin_amdgcn_s_waitcnt((4 & 15) | (7 << 4) | (15 << 8));  // vmcnt(4): the previous iteration's loads
    if (mode & 1) __builtin_amdgcn_s_barrier();
    if (mode & 2) {
      const int off = __builtin_amdgcn_readfirstlane(base + ((it * 8 + wave) & 15) * 4096);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (probe_lds_ptr)(smem + 96 * 1024 + (it & 1) * 32768 + (wave * 4 + u) * 1024), 16, lane * 16,
            off + u * 1024, 0, 0);
    }
    const int ro = (it & 3) * 8192;
    v4i bf[FN], af[3];
    af[0] = *(const v4i*)(sa + ro);
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[j] = *(const v4i*)(sb + j * 1024);
    af[1] = *(const v4i*)(sa + ro + 1024);
    __builtin_amdgcn_sched_group_barrier(0x100, FN + 2, 0);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if (i + 2 < FM) af[(i + 2) % 3] = *(const v4i*)(sa + ro + (i + 2) * 1024);
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i % 3], bf[j], acc[i][j], 0, 0, 0);
      if (i + 2 < FM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, FN, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8));
  v4i t = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) t += acc[i][j];
  if (t[0] == 0x7fffabcd) sink[threadIdx.x] = t[1] + smem[96 * 1024 + lane];
#endif
}

}  // namespace
}  // namespace fcmoe

using namespace fcmoe;

extern "C" int fcmoe_probe_stream(const void* src, int64_t src_bytes, int workgroups, int waves, int mode,
                                  int lds_pad_bytes, int* sink, hipStream_t stream) {
  if (!src || !sink || workgroups <= 0 || waves <= 0 || waves > 16 || (mode != 0 && mode != 1) || lds_pad_bytes < 0)
    return fail(FCMOE_EINVAL, "probe_stream: bad arguments");
  const int64_t chunks = src_bytes / 1024 / ((int64_t)workgroups * waves);
  if (chunks < 8) return fail(FCMOE_EINVAL, "probe_stream: fewer than 8 KiB per wave");
  const int lds = mode == 1 && lds_pad_bytes < waves * 8192 ? waves * 8192 : lds_pad_bytes;
  if (lds > 160 * 1024) return fail(FCMOE_EINVAL, "probe_stream: LDS beyond 160 KiB");
  static bool attr = false;
  if (!attr) {
    if (hipFuncSetAttribute((const void*)probe_stream_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024) != hipSuccess)
      return fail(FCMOE_EDEVICE, "probe_stream: hipFuncSetAttribute failed");
    attr = true;
  }
  hipLaunchKernelGGL(probe_stream_kernel, dim3(workgroups), dim3(waves * kWave), lds, stream, (const uint8_t*)src,
                     chunks, mode, sink);
  return check_launch("probe_stream");
}

extern "C" int fcmoe_probe_mfma(int tile, int waves, int workgroups, int iters, int* sink, hipStream_t stream) {
  if (!sink || workgroups <= 0 || iters <= 0) return fail(FCMOE_EINVAL, "probe_mfma: bad arguments");
  // tile: 0 = 128x96, 1 = 128x64, 2 = 96x80, 3 = 64x96, 4 = 64x64 (rows x channels of one wave)
  switch (tile * 100 + waves) {
    case 8: return launch_mfma<8, 6, 8>(workgroups, iters, sink, stream);
    case 4: return launch_mfma<8, 6, 4>(workgroups, iters, sink, stream);
    case 108: return launch_mfma<8, 4, 8>(workgroups, iters, sink, stream);
    case 112: return launch_mfma<8, 4, 12>(workgroups, iters, sink, stream);
    case 212: return launch_mfma<6, 5, 12>(workgroups, iters, sink, stream);
    case 312: return launch_mfma<4, 6, 12>(workgroups, iters, sink, stream);
    case 408: return launch_mfma<4, 4, 8>(workgroups, iters, sink, stream);
    case 416: return launch_mfma<4, 4, 16>(workgroups, iters, sink, stream);
    default: return fail(FCMOE_EINVAL, "probe_mfma: unsupported tile / waves pair");
  }
}

extern "C" int fcmoe_probe_mix(const void* src, int64_t src_bytes, int compute_waves, int stream_waves, int iters,
                               int stream_mfma, int* sink, hipStream_t stream) {
  const int w = compute_waves + stream_waves;
  if (!src || !sink || compute_waves < 0 || stream_waves < 0 || w <= 0 || w > 16 || iters < 0)
    return fail(FCMOE_EINVAL, "probe_mix: bad arguments");
  constexpr int kCus = 256;
  const int64_t chunks = stream_waves ? src_bytes / 1024 / ((int64_t)kCus * stream_waves) / 8 * 8 : 8;
  if (stream_waves && chunks < 8) return fail(FCMOE_EINVAL, "probe_mix: source too small");
  hipLaunchKernelGGL(probe_mix_kernel, dim3(kCus), dim3(w * kWave), 0, stream, (const uint8_t*)src, chunks,
                     compute_waves, stream_waves, iters, stream_mfma, sink);
  return check_launch("probe_mix");
}

extern "C" int fcmoe_probe_fence(const void* src, int64_t src_bytes, int workgroups, int waves, int release,
                                 int* counters, void* rows, hipStream_t stream) {
  if (!src || !counters || !rows || workgroups <= 0 || waves <= 0 || waves > 16)
    return fail(FCMOE_EINVAL, "probe_fence: bad arguments");
  const int64_t chunks = src_bytes / 1024 / ((int64_t)workgroups * waves);
  if (chunks < 8) return fail(FCMOE_EINVAL, "probe_fence: fewer than 8 KiB per wave");
  hipLaunchKernelGGL(probe_fence_kernel, dim3(workgroups), dim3(waves * kWave), 0, stream, (const uint8_t*)src,
                     chunks, release, counters, (v4i*)rows);
  return check_launch("probe_fence");
}

extern "C" int fcmoe_probe_ring(const void* src, int64_t src_bytes, const void* arows, int64_t arows_bytes,
                                int workgroups, int lookahead, int a_loads, int barrier, int* sink,
                                hipStream_t stream) {
  if (!src || !arows || !sink || workgroups <= 0) return fail(FCMOE_EINVAL, "probe_ring: bad arguments");
  // the kernel reads a 2 MiB window of arows per XCD: 16 MiB in all
  if (arows_bytes < ((int64_t)16 << 20)) return fail(FCMOE_EINVAL, "probe_ring: arows must hold at least 16 MiB");
  const int64_t chunks = src_bytes / ((int64_t)workgroups * 8 * 4 * 1024);
  if (chunks < 8 || chunks * 8 * 4 * 1024 > 0x7ffffff0) return fail(FCMOE_EINVAL, "probe_ring: bad source size");
  const dim3 g((unsigned)workgroups), b(512);
  const uint8_t* s = (const uint8_t*)src;
  const uint8_t* a = (const uint8_t*)arows;
  switch (lookahead * 100 + a_loads * 10 + (barrier ? 1 : 0)) {
    case 201: hipLaunchKernelGGL((probe_ring_kernel<2, 0, 1>), g, b, 0, stream, s, a, chunks, sink); break;
    case 221: hipLaunchKernelGGL((probe_ring_kernel<2, 2, 1>), g, b, 0, stream, s, a, chunks, sink); break;
    case 220: hipLaunchKernelGGL((probe_ring_kernel<2, 2, 0>), g, b, 0, stream, s, a, chunks, sink); break;
    case 421: hipLaunchKernelGGL((probe_ring_kernel<4, 2, 1>), g, b, 0, stream, s, a, chunks, sink); break;
    case 621: hipLaunchKernelGGL((probe_ring_kernel<6, 2, 1>), g, b, 0, stream, s, a, chunks, sink); break;
    default: return fail(FCMOE_EINVAL, "probe_ring: unsupported lookahead / A loads / barrier");
  }
  return check_launch("probe_ring");
}

extern "C" int fcmoe_probe_loop_dma(const void* src, int64_t src_bytes, int mode, int iters, int* sink,
                                    hipStream_t stream) {
  if (!src || !sink || src_bytes < (1 << 20) || iters <= 0 || mode < 0 || mode > 7)
    return fcmoe::fail(FCMOE_EINVAL, "probe_loop_dma: bad arguments");
  hipLaunchKernelGGL(fcmoe::probe_loop_dma_kernel, dim3(256), dim3(512), 0, stream, (const uint8_t*)src, mode, iters,
                     sink);
  return fcmoe::check_launch("probe_loop_dma");
}
