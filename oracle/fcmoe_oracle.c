/*
 * fcmoe_oracle.c -- CPU restatement of hearth-stone/fused_cpp's fused-MoE
 * arithmetic, used ONLY as a test oracle.
 *
 * TEST INFRASTRUCTURE. Nothing in fused_cpp_amd/ links, loads or calls this
 * file. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * use it, and only as the checker / the timed CPU baseline.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root). Floating-point operations are spelled out
 * one IEEE-754 binary32 operation at a time (explicit fmaf where the reference
 * uses a fused SVE instruction) and the file is compiled with
 * -ffp-contract=off, so results are bit-reproducible and comparable bit for
 * bit with the HIP kernels, which follow the same operation sequence.
 *
 * Pins (what checks each function; see tests/test_oracle_*.py):
 *  - orc_fexpa_exp_neg: table entries against exp2 (closed form) and the
 *    whole evaluator against libm exp (relative error < 2e-6 over the clamp
 *    range); FEXPA table rounding vs real Arm hardware is parity unpinned.
 *  - orc_quant_row_away / orc_quant_row_even: closed forms, ties, zero rows.
 *  - orc_route_build: brute force and the torch argsort-stable reference.
 *  - orc_w8a8_forward: the reference test's own per-token reference
 *    (tests/test_moe_w8a8.py:40-69) at its tolerance (atol 3e-6), plus exact
 *    int64 GEMM checks of both accumulator stages.
 *  - orc_i8gemm: the reference test closed form (tests/test_i8gemm.py:18-37),
 *    atol 0.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- bf16 helpers: csrc/moe/arm/i8mm_w8a8/kernels.cpp:190-198 ---------- */
static inline float orc_bf16_to_f32(uint16_t b) {
  uint32_t u = ((uint32_t)b) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round-to-nearest-even by integer bias, exactly as store_bf16 (no NaN case). */
uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---- FEXPA table: the 23-bit fraction of 2^(i/64), round-to-nearest ---- */
static uint32_t g_fexpa[64];
static int g_fexpa_ready = 0;

static void orc_fexpa_init(void) {
  if (g_fexpa_ready) return;
  for (int i = 0; i < 64; ++i) {
    long double v = exp2l((long double)i / 64.0L) * 8388608.0L; /* 2^23 */
    long long r = llroundl(v);
    g_fexpa[i] = (uint32_t)(r - 8388608LL);
  }
  g_fexpa_ready = 1;
}

uint32_t orc_fexpa_entry(int i) {
  orc_fexpa_init();
  return g_fexpa[i & 63];
}

/* FEXPA: bits[5:0] index the table, bits[13:6] become the exponent field. */
static inline float orc_fexpa(uint32_t bits) {
  uint32_t idx = bits & 63u;
  uint32_t ex = (bits >> 6) & 0xffu;
  return u2f((ex << 23) | g_fexpa[idx]);
}

/* exp(-gate) as exp_fexpa_neg: csrc/moe/arm/i8mm_w8a8/kernels.cpp:200-209. */
float orc_fexpa_exp_neg(float gate) {
  orc_fexpa_init();
  float x = fmaxf(fminf(-gate, 87.0f), -87.0f);
  float encoded = fmaf(x, 1.4426950216293335f, 196735.0f);
  float k = encoded - 196735.0f;
  float residual = fmaf(-k, 0.693145751953125f, x);
  residual = fmaf(-k, 1.428606765330187e-06f, residual);
  float scale = orc_fexpa(f2u(encoded));
  float poly = fmaf(residual, 0.5000003576278687f, 1.000003695487976f);
  return fmaf(scale, poly * residual, scale);
}

/* ---- activation row quantisation --------------------------------------- */
/* quantize_bf16_row: csrc/moe/arm/i8mm_w8a8/kernels.cpp:211-228.
 * max|x| -> scale = max/127 (1 if max == 0) -> q = rinta(clamp(x*(1/scale))).
 * rinta rounds half away from zero (C roundf). */
void orc_quant_row_away(const uint16_t* src, int n, int8_t* dst, float* scale_out) {
  float m = 0.0f;
  for (int i = 0; i < n; ++i) {
    float a = fabsf(orc_bf16_to_f32(src[i]));
    if (a > m) m = a;
  }
  float scale = m > 0.0f ? m / 127.0f : 1.0f;
  *scale_out = scale;
  float inv = 1.0f / scale;
  for (int i = 0; i < n; ++i) {
    float v = orc_bf16_to_f32(src[i]) * inv;
    v = fmaxf(fminf(v, 127.0f), -127.0f);
    dst[i] = (int8_t)(int)roundf(v);
  }
}

/* i8gemm activation quantisation, the generic form the reference's tests pin
 * (tests/test_i8gemm.py:25-28; csrc/i8gemm.cpp:368-392): q = rint(x / scale),
 * ties to even, clamp [-128, 127]. x is bf16 (is_f32 = 0) or fp32. */
void orc_quant_row_even(const void* src, int is_f32, int n, int8_t* dst, float* scale_out) {
  const uint16_t* b = (const uint16_t*)src;
  const float* f = (const float*)src;
  float m = 0.0f;
  for (int i = 0; i < n; ++i) {
    float v = is_f32 ? f[i] : orc_bf16_to_f32(b[i]);
    float a = fabsf(v);
    if (a > m) m = a;
  }
  float scale = m > 0.0f ? m / 127.0f : 1.0f;
  *scale_out = scale;
  for (int i = 0; i < n; ++i) {
    float v = is_f32 ? f[i] : orc_bf16_to_f32(b[i]);
    float q = rintf(v / scale);
    if (q < -128.0f) q = -128.0f;
    if (q > 127.0f) q = 127.0f;
    dst[i] = (int8_t)(int)q;
  }
}

/* Per-output-channel weight quantisation:
 * csrc/moe/arm/i8mm_w8a8/kernels.cpp:451-457 (torch round = ties to even). */
void orc_quant_weight_rows(const uint16_t* w, int64_t rows, int cols, int8_t* q, float* scales) {
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* src = w + r * cols;
    float m = 0.0f;
    for (int i = 0; i < cols; ++i) {
      float a = fabsf(orc_bf16_to_f32(src[i]));
      if (a > m) m = a;
    }
    float scale = m > 0.0f ? m / 127.0f : 1.0f;
    scales[r] = scale;
    for (int i = 0; i < cols; ++i) {
      float v = rintf(orc_bf16_to_f32(src[i]) / scale);
      v = fmaxf(fminf(v, 127.0f), -127.0f);
      q[r * cols + i] = (int8_t)(int)v;
    }
  }
}

/* ---- routing ------------------------------------------------------------ */
/* Route build: ascending flat route index per expert.
 * csrc/moe/arm/i8mm_w8a8/kernels.cpp:583-588 and
 * csrc/moe/arm/common/fused_moe_bf16_tiled.cpp:6454-6483.
 * Routes are the flattened [T, k(+1)] slots; slot k is the appended shared
 * expert (src/fused_cpp/moe/bf16_tiled.py:1007-1013) when shared_id >= 0.
 * Returns the number of invalid ids (which are not placed). */
int64_t orc_route_build(const int64_t* ids, int64_t tokens, int64_t top_k, int64_t experts, int64_t shared_id,
                        int64_t* counts, int64_t* offsets, int64_t* sorted_routes) {
  int64_t kt = top_k + (shared_id >= 0 ? 1 : 0);
  int64_t routes = tokens * kt;
  int64_t bad = 0;
  for (int64_t e = 0; e < experts; ++e) counts[e] = 0;
  for (int64_t r = 0; r < routes; ++r) {
    int64_t t = r / kt, s = r % kt;
    int64_t e = s < top_k ? ids[t * top_k + s] : shared_id;
    if (e < 0 || e >= experts) { ++bad; continue; }
    counts[e]++;
  }
  offsets[0] = 0;
  for (int64_t e = 0; e < experts; ++e) offsets[e + 1] = offsets[e] + counts[e];
  int64_t* fill = (int64_t*)calloc((size_t)experts, sizeof(int64_t));
  for (int64_t r = 0; r < routes; ++r) {
    int64_t t = r / kt, s = r % kt;
    int64_t e = s < top_k ? ids[t * top_k + s] : shared_id;
    if (e < 0 || e >= experts) continue;
    sorted_routes[offsets[e] + fill[e]++] = r;
  }
  free(fill);
  return bad;
}

/* ---- exact int8 dot product --------------------------------------------- */
static inline int32_t dot_i8(const int8_t* a, const int8_t* b, int n) {
  int32_t s = 0;
  for (int i = 0; i < n; ++i) s += (int32_t)a[i] * (int32_t)b[i];
  return s;
}

/* ---- W13 epilogue: csrc/moe/arm/i8mm_w8a8/kernels.cpp:230-246 ---------- */
static inline uint16_t w13_value(int32_t acc_g, int32_t acc_u, float xs, float sg, float su, float limit) {
  float gate = (float)acc_g * (xs * sg);
  float up = (float)acc_u * (xs * su);
  gate = fminf(gate, limit);
  up = fmaxf(fminf(up, limit), -limit);
  float e = orc_fexpa_exp_neg(gate);
  float v = (gate * up) / (e + 1.0f);
  return orc_f32_to_bf16(v);
}

/* One route row after its W13 GEMM: w13_epilogue (kernels.cpp:230-246) over
 * the I gate/up pairs, then quantize_bf16_row of the bf16 row (:211-228,
 * :650-657). */
static void w13_row(const int32_t* a13, int I, float xs, const float* se, uint16_t* y, int8_t* q2, float* s2r) {
  for (int f = 0; f < I; ++f) y[f] = w13_value(a13[f], a13[I + f], xs, se[f], se[I + f], 10.0f);
  orc_quant_row_away(y, I, q2, s2r);
}

/* store_w2 (kernels.cpp:248-257): route row = (float)acc * (s_row * s_w). */
static inline float w2_value(int32_t acc, float s2r, float sw) { return (float)acc * (s2r * sw); }

/* Merge (kernels.cpp:674-688): per token and channel acc = fma(route, w, acc)
 * over the kt slots in slot order, then bf16. */
static void merge_rows(const float* route_out, const float* rw, int64_t tokens, int64_t kt, int64_t hidden,
                       uint16_t* out) {
  int64_t t;
#pragma omp parallel for schedule(static)
  for (t = 0; t < tokens; ++t) {
    for (int64_t h = 0; h < hidden; ++h) {
      float acc = 0.0f;
      for (int64_t s = 0; s < kt; ++s) {
        const int64_t r = t * kt + s;
        acc = fmaf(route_out[r * hidden + h], rw[r], acc);
      }
      out[t * hidden + h] = orc_f32_to_bf16(acc);
    }
  }
}

/* The forward's stages after each GEMM, for checking a whole layer whose
 * int32 accumulators come from an exact integer GEMM elsewhere (the same
 * arithmetic as orc_w8a8_forward, which calls the same helpers):
 * orc_w8a8_w13_rows: rows route rows of one expert, acc13 [rows, 2I], xs [rows]
 *   (the rows' token scales), s13e [2I] -> q2 [rows, I], s2row [rows]
 *   (y [rows, I] bf16 bits when not NULL);
 * orc_w8a8_w2_rows: acc2 [rows, H], s2row [rows], s2e [H] -> route_out [rows, H];
 * orc_w8a8_merge: route_out [T * kt, H] by flat route, rw [T * kt] -> out [T, H]. */
void orc_w8a8_w13_rows(const int32_t* acc13, int64_t rows, int64_t inter, const float* xs, const float* s13e,
                       uint16_t* y_out, int8_t* q2, float* s2row) {
  int64_t j;
#pragma omp parallel for schedule(static)
  for (j = 0; j < rows; ++j) {
    uint16_t* y = y_out ? y_out + j * inter : (uint16_t*)malloc((size_t)inter * sizeof(uint16_t));
    w13_row(acc13 + j * 2 * inter, (int)inter, xs[j], s13e, y, q2 + j * inter, s2row + j);
    if (!y_out) free(y);
  }
}

void orc_w8a8_w2_rows(const int32_t* acc2, int64_t rows, int64_t hidden, const float* s2row, const float* s2e,
                      float* route_out) {
  int64_t j;
#pragma omp parallel for schedule(static)
  for (j = 0; j < rows; ++j)
    for (int64_t h = 0; h < hidden; ++h) route_out[j * hidden + h] = w2_value(acc2[j * hidden + h], s2row[j], s2e[h]);
}

void orc_w8a8_merge(const float* route_out, const float* rw, int64_t tokens, int64_t kt, int64_t hidden,
                    uint16_t* out) {
  merge_rows(route_out, rw, tokens, kt, hidden, out);
}

/* Full W8A8 fused-MoE forward, csrc/moe/arm/i8mm_w8a8/kernels.cpp:463-694:
 * per route row: quantize_bf16_row(x[token]) -> W13 int32 GEMM -> w13_epilogue
 * (clamped SwiGLU, bf16) -> quantize_bf16_row -> W2 int32 GEMM -> store_w2
 * (acc * (s_row * s_w2)) -> per-token ordered FMA merge over slots -> bf16.
 *
 * Layout: x [T,H] bf16; ids [T,k] int64; topk_w [T,k] fp32;
 * w13 [E, 2I, H] int8, s13 [E, 2I]; w2 [E, H, I] int8, s2 [E, H].
 * shared_id >= 0 appends slot k with expert shared_id and weight 1.0; routed
 * weights are multiplied by routed_scale (bf16_tiled.py:1007-1013).
 * Optional dumps (NULL to skip), all indexed by flat route r in [0, T*kt):
 *   acc13 [R, 2I] int32, y [R, I] bf16 bits, q2 [R, I] int8, s2row [R],
 *   acc2 [R, H] int32, route_out [R, H] fp32.
 * out [T, H] bf16 bits. Routes with invalid ids contribute nothing. */
void orc_w8a8_forward(const uint16_t* x, const int64_t* ids, const float* topk_w, int64_t tokens, int64_t top_k,
                      int64_t hidden, int64_t inter, int64_t experts, const int8_t* w13, const float* s13,
                      const int8_t* w2, const float* s2, int64_t shared_id, float routed_scale, uint16_t* out,
                      int32_t* d_acc13, uint16_t* d_y, int8_t* d_q2, float* d_s2row, int32_t* d_acc2,
                      float* d_route) {
  const int64_t kt = top_k + (shared_id >= 0 ? 1 : 0);
  const int64_t routes = tokens * kt;
  const int H = (int)hidden, I = (int)inter;
  float* route_out = (float*)calloc((size_t)(routes * hidden), sizeof(float));
  float* rw = (float*)malloc((size_t)routes * sizeof(float));
  int64_t t;
#pragma omp parallel for schedule(dynamic, 1)
  for (t = 0; t < tokens; ++t) {
    int8_t* xq = (int8_t*)malloc((size_t)H);
    int32_t* a13 = (int32_t*)malloc((size_t)(2 * I) * sizeof(int32_t));
    uint16_t* y = (uint16_t*)malloc((size_t)I * sizeof(uint16_t));
    int8_t* q2 = (int8_t*)malloc((size_t)I);
    float xs;
    orc_quant_row_away(x + t * hidden, H, xq, &xs);
    for (int64_t s = 0; s < kt; ++s) {
      const int64_t r = t * kt + s;
      int64_t e = s < top_k ? ids[t * top_k + s] : shared_id;
      rw[r] = s < top_k ? (shared_id >= 0 ? topk_w[t * top_k + s] * routed_scale : topk_w[t * top_k + s]) : 1.0f;
      if (e < 0 || e >= experts) continue;
      const int8_t* we = w13 + (size_t)e * 2 * I * H;
      for (int n = 0; n < 2 * I; ++n) a13[n] = dot_i8(xq, we + (size_t)n * H, H);
      float s2r;
      w13_row(a13, I, xs, s13 + (size_t)e * 2 * I, y, q2, &s2r);
      const int8_t* w2e = w2 + (size_t)e * H * I;
      const float* s2e = s2 + (size_t)e * H;
      float* ro = route_out + r * hidden;
      for (int h = 0; h < H; ++h) {
        int32_t acc = dot_i8(q2, w2e + (size_t)h * I, I);
        if (d_acc2) d_acc2[r * hidden + h] = acc;
        ro[h] = w2_value(acc, s2r, s2e[h]);
      }
      if (d_acc13) memcpy(d_acc13 + r * 2 * I, a13, (size_t)(2 * I) * sizeof(int32_t));
      if (d_y) memcpy(d_y + r * I, y, (size_t)I * sizeof(uint16_t));
      if (d_q2) memcpy(d_q2 + r * I, q2, (size_t)I);
      if (d_s2row) d_s2row[r] = s2r;
    }
    free(xq); free(a13); free(y); free(q2);
  }
  /* Merge: kernels.cpp:674-688 -- acc = fma(route, w, acc) in slot order. */
  merge_rows(route_out, rw, tokens, kt, hidden, out);
  if (d_route) memcpy(d_route, route_out, (size_t)(routes * hidden) * sizeof(float));
  free(route_out);
  free(rw);
}

/* Grouped W8A8 layer throughput form used as the timed CPU baseline: the same
 * arithmetic as orc_w8a8_forward but grouped per expert (each expert's routed
 * rows against its weights), which is the cache-friendly order a CPU
 * implementation uses (kernels.cpp:627-689 processes one expert task at a time).
 * Processes only experts [e_begin, e_end) and writes route_out rows for them;
 * the caller merges. Returns the number of routed rows processed. */
int64_t orc_w8a8_expert_range(const uint16_t* x, const int64_t* sorted_routes, const int64_t* offsets, int64_t kt,
                              int64_t hidden, int64_t inter, const int8_t* w13, const float* s13, const int8_t* w2,
                              const float* s2, int64_t e_begin, int64_t e_end, float* route_out) {
  const int H = (int)hidden, I = (int)inter;
  int64_t done = 0;
  for (int64_t e = e_begin; e < e_end; ++e) {
    const int64_t rows = offsets[e + 1] - offsets[e];
    done += rows;
    int64_t j;
#pragma omp parallel for schedule(dynamic, 1)
    for (j = 0; j < rows; ++j) {
      const int64_t r = sorted_routes[offsets[e] + j];
      const int64_t t = r / kt;
      int8_t* xq = (int8_t*)malloc((size_t)H);
      int32_t* a13 = (int32_t*)malloc((size_t)(2 * I) * sizeof(int32_t));
      uint16_t* y = (uint16_t*)malloc((size_t)I * sizeof(uint16_t));
      int8_t* q2 = (int8_t*)malloc((size_t)I);
      float xs, s2r;
      orc_quant_row_away(x + t * hidden, H, xq, &xs);
      const int8_t* we = w13 + (size_t)e * 2 * I * H;
      for (int n = 0; n < 2 * I; ++n) a13[n] = dot_i8(xq, we + (size_t)n * H, H);
      w13_row(a13, I, xs, s13 + (size_t)e * 2 * I, y, q2, &s2r);
      const int8_t* w2e = w2 + (size_t)e * H * I;
      const float* s2e = s2 + (size_t)e * H;
      float* ro = route_out + r * hidden;
      for (int h = 0; h < H; ++h) ro[h] = w2_value(dot_i8(q2, w2e + (size_t)h * I, I), s2r, s2e[h]);
      free(xq); free(a13); free(y); free(q2);
    }
  }
  return done;
}

/* Exact grouped int32 GEMM of gathered int8 rows against one expert's [N, K]
 * int8 weight: acc[j, n] = sum_k a[rows[j], k] * w[e][n, k]. Used to check the
 * GPU accumulator stages bit for bit on identical int8 operands. */
void orc_gemm_i8_rows(const int8_t* a, int64_t lda, const int64_t* rows, int64_t nrows, const int8_t* w, int64_t n,
                      int64_t k, int32_t* acc) {
  int64_t j;
#pragma omp parallel for schedule(static)
  for (j = 0; j < nrows; ++j) {
    const int8_t* ar = a + rows[j] * lda;
    for (int64_t c = 0; c < n; ++c) acc[j * n + c] = dot_i8(ar, w + c * k, (int)k);
  }
}

/* i8gemm.dynamic_scaled_mm, the generic semantics
 * (csrc/i8gemm.cpp:368-392 quantisation, :148-164 write_scaled_output):
 * out = (float)acc * x_scale * w_scale[n] (left to right) + bias[n];
 * out_bf16 != 0 stores bf16 RNE bits, else fp32. */
void orc_i8gemm(const void* x, int x_is_f32, int64_t m, int64_t k, const int8_t* w, const float* w_scale, int64_t n,
                const float* bias, int out_bf16, void* out) {
  int64_t r;
#pragma omp parallel for schedule(static)
  for (r = 0; r < m; ++r) {
    int8_t* q = (int8_t*)malloc((size_t)k);
    float xs;
    const char* src = (const char*)x + r * k * (x_is_f32 ? 4 : 2);
    orc_quant_row_even(src, x_is_f32, (int)k, q, &xs);
    for (int64_t c = 0; c < n; ++c) {
      int32_t acc = dot_i8(q, w + c * k, (int)k);
      float v = (float)acc * xs * w_scale[c];
      if (bias) v = v + bias[c];
      if (out_bf16)
        ((uint16_t*)out)[r * n + c] = orc_f32_to_bf16(v);
      else
        ((float*)out)[r * n + c] = v;
    }
    free(q);
  }
}

/* BF16 W13 activation epilogues (fp32 in, bf16 out), the semantics of
 * csrc/moe/arm/common/fused_moe_bf16_tiled.cpp:1861-1914 and the limit-10
 * clamp of src/fused_cpp/moe/bf16_tiled.py:245-260:
 * mode 0 silu, 1 gelu (erf), 2 swigluoai (interleaved), 3 silu clamp 10.
 * gate_up [rows, 2F]; y [rows, F] bf16 bits. Uses libm expf/erff, so this is
 * a tolerance reference for the GPU (which uses its own expf/erff). */
void orc_bf16_activation(const float* gate_up, int64_t rows, int64_t f, int mode, uint16_t* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* g = gate_up + r * 2 * f;
    for (int64_t c = 0; c < f; ++c) {
      float v;
      if (mode == 2) {
        float gate = fminf(g[2 * c], 7.0f);
        float up = fmaxf(-7.0f, fminf(g[2 * c + 1], 7.0f));
        float glu = gate / (1.0f + expf(-gate * 1.702f));
        v = (up + 1.0f) * glu;
      } else {
        float gate = g[c], up = g[f + c];
        if (mode == 3) {
          gate = fminf(gate, 10.0f);
          up = fmaxf(fminf(up, 10.0f), -10.0f);
        }
        if (mode == 1)
          v = 0.5f * gate * (1.0f + erff(gate * 0.70710678118654752440f)) * up;
        else
          v = gate / (1.0f + expf(-gate)) * up;
      }
      y[r * f + c] = orc_f32_to_bf16(v);
    }
  }
}

/* ---- BF16 top-k merge (csrc/moe/arm/sve_bf16/route_merge.cpp:38-126) ----
 * route_out rows are indexed by flat route t*kt + s. For kt in {2, 4, 6, 8}
 * the SVE merge multiplies each row by its weight (weighted_leaf, :47-52) and
 * adds the products as a tree that splits every range at the largest power of
 * two below its length (reduce_fixed, :54-69): ((0+1)+(2+3))+(4+5) for 6.
 * Other kt: acc = 0, then acc = fma(row_s, w_s, acc) for s = 0..kt-1
 * (merge_dynamic_block, :78-86; svmla is a fused multiply-add). The fp32 sum
 * is rounded to bf16 to nearest even. */
static int orc_pow2_below(int n) {
  int p = 1;
  while ((p << 1) < n) p <<= 1;
  return p;
}

static float orc_tree(const float* leaf, int begin, int count) {
  if (count == 1) return leaf[begin];
  const int left = orc_pow2_below(count);
  const float a = orc_tree(leaf, begin, left);
  const float b = orc_tree(leaf, begin + left, count - left);
  return a + b;
}

void orc_bf16_route_merge(const float* route_out, const float* weights, int64_t tokens, int64_t kt, int64_t hidden,
                          uint16_t* out) {
  const int tree = kt == 2 || kt == 4 || kt == 6 || kt == 8;
  for (int64_t t = 0; t < tokens; ++t) {
    for (int64_t h = 0; h < hidden; ++h) {
      float acc = 0.0f;
      if (tree) {
        float leaf[8];
        for (int64_t s = 0; s < kt; ++s) leaf[s] = route_out[(t * kt + s) * hidden + h] * weights[t * kt + s];
        acc = orc_tree(leaf, 0, (int)kt);
      } else {
        for (int64_t s = 0; s < kt; ++s) acc = fmaf(route_out[(t * kt + s) * hidden + h], weights[t * kt + s], acc);
      }
      out[t * hidden + h] = orc_f32_to_bf16(acc);
    }
  }
}
