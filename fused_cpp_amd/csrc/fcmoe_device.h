// fcmoe_device.h -- gfx950 device helpers shared by the fused-MoE kernels.
//
// Every floating-point helper spells out one binary32 operation at a time
// (the library is compiled with -ffp-contract=off), so the W8A8 path produces
// the same bits as the CPU restatement of the reference arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fcmoe {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// Round-to-nearest-even by integer bias, as store_bf16
// (csrc/moe/arm/i8mm_w8a8/kernels.cpp:194-198); no NaN special case.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

// 23-bit fractions of 2^(i/64), rounded to nearest: the FEXPA coefficient
// table that exp_fexpa_neg (csrc/moe/arm/i8mm_w8a8/kernels.cpp:200-209)
// relies on. Generated from exp2 and checked against it in the CPU tests.
__constant__ static const uint32_t kFexpaTable[64] = {
    0x000000, 0x0164d2, 0x02cd87, 0x043a29, 0x05aac3, 0x071f62, 0x08980f, 0x0a14d5, 0x0b95c2, 0x0d1adf, 0x0ea43a,
    0x1031dc, 0x11c3d3, 0x135a2b, 0x14f4f0, 0x16942d, 0x1837f0, 0x19e046, 0x1b8d3a, 0x1d3eda, 0x1ef532, 0x20b051,
    0x227043, 0x243516, 0x25fed7, 0x27cd94, 0x29a15b, 0x2b7a3a, 0x2d583f, 0x2f3b79, 0x3123f6, 0x3311c4, 0x3504f3,
    0x36fd92, 0x38fbaf, 0x3aff5b, 0x3d08a4, 0x3f179a, 0x412c4d, 0x4346cd, 0x45672a, 0x478d75, 0x49b9be, 0x4bec15,
    0x4e248c, 0x506334, 0x52a81e, 0x54f35b, 0x5744fd, 0x599d16, 0x5bfbb8, 0x5e60f5, 0x60ccdf, 0x633f89, 0x65b907,
    0x68396a, 0x6ac0c7, 0x6d4f30, 0x6fe4ba, 0x728177, 0x75257d, 0x77d0df, 0x7a83b3, 0x7d3e0c};

// exp(-gate) evaluated exactly as exp_fexpa_neg
// (csrc/moe/arm/i8mm_w8a8/kernels.cpp:200-209): clamp, shift-encode,
// two-step Cody-Waite residual, FEXPA scale, degree-2 polynomial.
// The table held in one VGPR, entry i in lane i (load once per kernel):
// lookups then go through the LDS crossbar (ds_bpermute) instead of a
// divergent __constant__ load that waits on the memory pipeline.
__device__ __forceinline__ uint32_t fexpa_table_lane() { return kFexpaTable[threadIdx.x % kWave]; }

// exp_fexpa_neg with the table in a VGPR (fexpa_table_lane), split so a
// caller can issue many lookups before it waits for any: fexpa_reduce computes
// the argument's encoding and residual, fexpa_lookup reads the table entry
// (ds_bpermute, all lanes active), fexpa_finish forms the result. Together
// they give exactly fexpa_exp_neg's bits.
struct FexpaArg {
  uint32_t bits;   // encoded value's bits: exponent in [13:6], table index in [5:0]
  float residual;
};
__device__ __forceinline__ FexpaArg fexpa_reduce(float gate) {
  float x = fmaxf(fminf(-gate, 87.0f), -87.0f);
  float encoded = __builtin_fmaf(x, 1.4426950216293335f, 196735.0f);
  float k = encoded - 196735.0f;
  float residual = __builtin_fmaf(-k, 0.693145751953125f, x);
  residual = __builtin_fmaf(-k, 1.428606765330187e-06f, residual);
  return FexpaArg{__float_as_uint(encoded), residual};
}
__device__ __forceinline__ uint32_t fexpa_lookup(uint32_t bits, uint32_t tab) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute((int)((bits & 63u) << 2), (int)tab);
}
__device__ __forceinline__ float fexpa_finish(FexpaArg a, uint32_t frac) {
  float scale = __uint_as_float((((a.bits >> 6) & 0xffu) << 23) | frac);
  float poly = __builtin_fmaf(a.residual, 0.5000003576278687f, 1.000003695487976f);
  return __builtin_fmaf(scale, poly * a.residual, scale);
}
__device__ __forceinline__ float fexpa_exp_neg_v(float gate, uint32_t tab) {
  const FexpaArg a = fexpa_reduce(gate);
  return fexpa_finish(a, fexpa_lookup(a.bits, tab));
}

__device__ __forceinline__ float fexpa_exp_neg(float gate) {
  float x = fmaxf(fminf(-gate, 87.0f), -87.0f);
  float encoded = __builtin_fmaf(x, 1.4426950216293335f, 196735.0f);
  float k = encoded - 196735.0f;
  float residual = __builtin_fmaf(-k, 0.693145751953125f, x);
  residual = __builtin_fmaf(-k, 1.428606765330187e-06f, residual);
  uint32_t bits = __float_as_uint(encoded);
  float scale = __uint_as_float((((bits >> 6) & 0xffu) << 23) | kFexpaTable[bits & 63u]);
  float poly = __builtin_fmaf(residual, 0.5000003576278687f, 1.000003695487976f);
  return __builtin_fmaf(scale, poly * residual, scale);
}

// Max over the 16 lanes that share (lane / 16) -- one DPP row -- with DPP
// moves (no LDS crossbar): quad max via quad_perm [1,0,3,2] and [2,3,0,1],
// then rotations of the row by 4 and 8 lanes fold in the other quads. Every
// lane ends with the row maximum (max is exact in any order).
// mov_dpp (no old operand; every source lane here lies inside the row) lets
// the compiler fold the move into the v_max that consumes it (v_max_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}
// The invalid-id count: a relaxed store at system scope (a vector store that
// goes through to memory), so that a host polling pinned memory for it sees
// it while the kernel is still running rather than at the kernel's end.
__device__ __forceinline__ void store_count(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp_f<0x128>(v));  // row_ror:8
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ int wave_sum(int v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Butterfly sum: every lane ends with the same value (same pairing order).
__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__host__ __device__ __forceinline__ int64_t round_up(int64_t v, int64_t q) { return (v + q - 1) / q * q; }
__host__ __device__ __forceinline__ int64_t ceil_div(int64_t v, int64_t q) { return (v + q - 1) / q; }

}  // namespace fcmoe
