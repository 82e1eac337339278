/*
 * pf_oracle.c — CPU restatement of textsift's WASM forward (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker / CPU baseline. Never linked
 * into the product library.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off). The no-contraction
 * flag matters: the reference rounds every multiply and add separately
 * except at relaxed_madd sites (c/fma.c:10-13), which are written here as
 * explicit fmaf() calls.
 *
 * Citations are into /root/reference/packages/textsift/src/.
 *
 * Parity status of each part (what pins it is in tests/test_oracle_*.py):
 *   conversions, int4 decode, embed, matmul, rms/add-rms norms, topk, rope,
 *   attention, swiglu, scatter/cast: pinned by the reference's conformance
 *   fixtures plus closed forms / exhaustive sweeps.
 *   expf standing in for Zig's std @exp (softmax_f32, scalar sigmoid tail,
 *   attention scalar tail): parity unpinned at the last ulp.
 */
#include "pf_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* conversions — zig/math.zig                                          */
/* ------------------------------------------------------------------ */

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* zig/math.zig:45-52 fp16ToF32 (and the vector form :84-103): not IEEE for
 * subnormals / inf / NaN — the exponent rebias is applied blindly. */
static inline float h2f(uint16_t bits) {
  uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
  uint32_t rest = (uint32_t)bits & 0x7fffu;
  uint32_t biased = rest == 0 ? 0u : (rest << 13) + (112u << 23);
  return bits_f32(sign | biased);
}

/* zig/math.zig:54-82 f32ToFp16: RNE for normals, round-half-up for
 * subnormals, overflow -> inf, NaN keeps a quiet bit. */
static inline uint16_t f2h(float f) {
  uint32_t u = f32_bits(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t exp32 = (u >> 23) & 0xffu;
  uint32_t mant = u & 0x7fffffu;
  if (exp32 == 0xffu) return (uint16_t)(sign | 0x7c00u | (mant != 0 ? 0x200u : 0u));
  int32_t e16 = (int32_t)exp32 - 127 + 15;
  if (e16 >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (e16 <= 0) {
    if (e16 < -10) return (uint16_t)sign;
    uint32_t shift = (uint32_t)(14 - e16);
    uint32_t mant24 = mant | 0x800000u;
    uint32_t rounded = (mant24 + (1u << (shift - 1))) >> shift;
    return (uint16_t)(sign | rounded);
  }
  uint32_t lsb = (mant >> 13) & 1u;
  uint32_t m10 = (mant + 0xfffu + lsb) >> 13;
  uint32_t e = (uint32_t)e16;
  if (m10 >= 0x400u) {
    m10 = 0;
    e += 1;
    if (e >= 0x1fu) return (uint16_t)(sign | 0x7c00u);
  }
  return (uint16_t)(sign | (e << 10) | m10);
}

float pfo_fp16_to_f32(uint16_t h) { return h2f(h); }
uint16_t pfo_f32_to_fp16(float f) { return f2h(f); }
void pfo_fp16_to_f32_n(const uint16_t* s, float* d, size_t n) { for (size_t i = 0; i < n; i++) d[i] = h2f(s[i]); }
void pfo_f32_to_fp16_n(const float* s, uint16_t* d, size_t n) { for (size_t i = 0; i < n; i++) d[i] = f2h(s[i]); }

/* ------------------------------------------------------------------ */
/* approximate exp / sigmoid — zig/wasm_exports.zig:794-853            */
/* ------------------------------------------------------------------ */

/* expApproxNonPositiveF32x4 (:812-838), one lane. */
static inline float exp_approx(float x) {
  const float LOG2_E = 1.44269504088896340736f;
  float clamped = fmaxf(x, -88.0f);
  float y = clamped * LOG2_E;
  int32_t iv = (int32_t)floorf(y);
  float frac = y - (float)iv;
  float poly = fmaf(0.001333355f, frac, 0.009679494f);
  poly = fmaf(poly, frac, 0.055053319f);
  poly = fmaf(poly, frac, 0.240226522f);
  poly = fmaf(poly, frac, 0.693154774f);
  poly = fmaf(poly, frac, 1.000000012f);
  float scale = bits_f32((uint32_t)(iv + 127) << 23);
  return poly * scale;
}
float pfo_exp_approx(float x) { return exp_approx(x); }

/* sigmoidF32x4 (:843-853), one lane. */
static inline float sigmoid_approx(float x) {
  float neg_abs = fminf(x, 0.0f) - fmaxf(x, 0.0f);
  float e = exp_approx(neg_abs);
  float sig_neg = e / (1.0f + e);
  return x >= 0.0f ? 1.0f - sig_neg : sig_neg;
}

/* sigmoidF32 (:794-804) — scalar tail; Zig @exp stood in by expf. */
static inline float sigmoid_scalar(float x) {
  if (x >= 0.0f) {
    float e = expf(-x);
    return 1.0f / (1.0f + e);
  }
  float e = expf(x);
  return e / (1.0f + e);
}

/* ------------------------------------------------------------------ */
/* norms — :186-350                                                    */
/* ------------------------------------------------------------------ */

void pfo_rms_norm(const uint16_t* x, const uint16_t* g, uint16_t* out, uint32_t T, uint32_t D, float eps) {
  const float d_inv = 1.0f / (float)D;
  for (uint32_t t = 0; t < T; t++) {
    const uint16_t* xr = x + (size_t)t * D;
    float sumsq = 0.0f;
    for (uint32_t d = 0; d < D; d++) { float v = h2f(xr[d]); sumsq += v * v; }
    float inv_rms = 1.0f / sqrtf(sumsq * d_inv + eps);
    for (uint32_t d = 0; d < D; d++) out[(size_t)t * D + d] = f2h(h2f(xr[d]) * inv_rms * h2f(g[d]));
  }
}

/* 4-lane partial sums of squares, lanes combined left to right (:236-248). */
static inline float sumsq4(const float* v, uint32_t D) {
  float s[4] = {0, 0, 0, 0};
  uint32_t d = 0;
  for (; d + 4 <= D; d += 4)
    for (int c = 0; c < 4; c++) s[c] += v[d + c] * v[d + c];
  float r = s[0] + s[1] + s[2] + s[3];
  for (; d < D; d++) r += v[d] * v[d];
  return r;
}

void pfo_rms_norm_fp16_to_f32(const uint16_t* x, const uint16_t* g, float* out, uint32_t T, uint32_t D, float eps) {
  const float d_inv = 1.0f / (float)D;
  float* row = (float*)malloc(sizeof(float) * D);
  for (uint32_t t = 0; t < T; t++) {
    const uint16_t* xr = x + (size_t)t * D;
    for (uint32_t d = 0; d < D; d++) row[d] = h2f(xr[d]);
    float inv_rms = 1.0f / sqrtf(sumsq4(row, D) * d_inv + eps);
    float* o = out + (size_t)t * D;
    for (uint32_t d = 0; d < D; d++) o[d] = row[d] * inv_rms * h2f(g[d]);
  }
  free(row);
}

void pfo_add_rmsnorm_fp16_to_f32(const uint16_t* a, const uint16_t* b, const uint16_t* g, uint16_t* sum_out,
                                 float* norm_out, uint32_t T, uint32_t D, float eps) {
  const float d_inv = 1.0f / (float)D;
  float* row = (float*)malloc(sizeof(float) * D);
  for (uint32_t t = 0; t < T; t++) {
    const size_t base = (size_t)t * D;
    for (uint32_t d = 0; d < D; d++) {
      row[d] = h2f(a[base + d]) + h2f(b[base + d]);
      sum_out[base + d] = f2h(row[d]);
    }
    /* sumsq is taken on the unrounded f32 sum (:312-320) */
    float inv_rms = 1.0f / sqrtf(sumsq4(row, D) * d_inv + eps);
    /* pass 2 re-reads the fp16-rounded sum (:332-345) */
    for (uint32_t d = 0; d < D; d++) norm_out[base + d] = h2f(sum_out[base + d]) * inv_rms * h2f(g[d]);
  }
  free(row);
}

/* ------------------------------------------------------------------ */
/* top-k — :367-426                                                    */
/* ------------------------------------------------------------------ */

void pfo_topk_partial_f32(const float* x, int32_t* oi, float* ov, uint32_t rows, uint32_t cols, uint32_t k) {
  for (uint32_t r = 0; r < rows; r++) {
    const float* xr = x + (size_t)r * cols;
    int32_t* I = oi + (size_t)r * k;
    float* V = ov + (size_t)r * k;
    for (uint32_t i = 0; i < k; i++) { I[i] = (int32_t)i; V[i] = xr[i]; }
    for (uint32_t s = 1; s < k; s++) {
      for (uint32_t j = s; j > 0 && V[j] > V[j - 1]; j--) {
        float tv = V[j]; V[j] = V[j - 1]; V[j - 1] = tv;
        int32_t ti = I[j]; I[j] = I[j - 1]; I[j - 1] = ti;
      }
    }
    for (uint32_t c = k; c < cols; c++) {
      float v = xr[c];
      if (v > V[k - 1]) {
        V[k - 1] = v;
        I[k - 1] = (int32_t)c;
        for (uint32_t j = k - 1; j > 0 && V[j] > V[j - 1]; j--) {
          float tv = V[j]; V[j] = V[j - 1]; V[j - 1] = tv;
          int32_t ti = I[j]; I[j] = I[j - 1]; I[j - 1] = ti;
        }
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* int4 MatMulNBits — :458-766                                         */
/* ------------------------------------------------------------------ */

/* int4BlockDecode (:507-536): element j of the block = nibble (j&1) of byte
 * j/2 (low nibble first), minus zp, as an exact float. */
static inline void decode_block(const uint8_t* row, size_t block_d, uint32_t zp, float q[32]) {
  const uint8_t* p = row + block_d / 2;
  for (int j = 0; j < 16; j++) {
    q[2 * j] = (float)((int)(p[j] & 0x0f) - (int)zp);
    q[2 * j + 1] = (float)((int)(p[j] >> 4) - (int)zp);
  }
}

/* extractZp (:541-544) */
static inline uint32_t extract_zp(const uint8_t* zp_row, size_t b) {
  uint8_t byte = zp_row[b >> 1];
  return (b & 1) == 0 ? (byte & 0x0fu) : ((byte >> 4) & 0x0fu);
}

static inline float load_x(int x_f32, const void* x, size_t i) {
  return x_f32 ? ((const float*)x)[i] : h2f(((const uint16_t*)x)[i]);
}

static inline void store_out(int out_f32, void* out, size_t i, float v) {
  if (out_f32) ((float*)out)[i] = v;
  else ((uint16_t*)out)[i] = f2h(v);
}

void pfo_matmul_int4block(int x_f32, int out_f32, const void* x, const uint8_t* w_int4, const uint16_t* w_scales,
                          const uint8_t* w_zp, const uint16_t* bias, void* out, uint32_t T, uint32_t N,
                          uint32_t D) {
  const size_t Dz = D, Nz = N;
  const size_t BLOCK = 32, TR = 8;
  const size_t w_stride = Dz / 2;
  const size_t s_stride = Dz / BLOCK;
  const size_t z_stride = (s_stride + 1) / 2;
  float q[32];
  size_t tt = 0;
  /* TR=8 main path (:589-662): per row, 4 lanes x 8 sequential FMAs per
   * block (lane c takes elements c, c+4, ..., c+28), then
   * (l0+l1)+(l2+l3), then sum += blk*scale (two roundings). */
  for (; tt + TR <= T; tt += TR) {
    for (size_t n = 0; n < Nz; n++) {
      const uint8_t* wrow = w_int4 + n * w_stride;
      const uint16_t* srow = w_scales + n * s_stride;
      const uint8_t* zrow = w_zp ? w_zp + n * z_stride : NULL;
      float sum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (size_t b = 0; b < s_stride; b++) {
        const float scale = h2f(srow[b]);
        const size_t bd = b * BLOCK;
        decode_block(wrow, bd, zrow ? extract_zp(zrow, b) : 0u, q);
        for (size_t r = 0; r < TR; r++) {
          const size_t xb = (tt + r) * Dz + bd;
          float v[4] = {0, 0, 0, 0};
          for (int k = 0; k < 4; k++) {
            const int j = k * 8;
            for (int c = 0; c < 4; c++) v[c] = fmaf(load_x(x_f32, x, xb + j + c), q[j + c], v[c]);
            for (int c = 0; c < 4; c++) v[c] = fmaf(load_x(x_f32, x, xb + j + 4 + c), q[j + 4 + c], v[c]);
          }
          const float blk = (v[0] + v[1]) + (v[2] + v[3]);
          const float prod = blk * scale;
          sum[r] = sum[r] + prod;
        }
      }
      const float bv = h2f(bias[n]);
      for (size_t r = 0; r < TR; r++) store_out(out_f32, out, (tt + r) * Nz + n, sum[r] + bv);
    }
  }
  /* T tail (:669-707): two 4-lane accumulators over alternating chunks,
   * combined lane-wise, then reduced and scaled per block. */
  const size_t m_tail = T - tt;
  if (m_tail > 0) {
    for (size_t n = 0; n < Nz; n++) {
      const uint8_t* wrow = w_int4 + n * w_stride;
      const uint16_t* srow = w_scales + n * s_stride;
      const uint8_t* zrow = w_zp ? w_zp + n * z_stride : NULL;
      float accs[7] = {0, 0, 0, 0, 0, 0, 0};
      for (size_t b = 0; b < s_stride; b++) {
        const float scale = h2f(srow[b]);
        const size_t bd = b * BLOCK;
        decode_block(wrow, bd, zrow ? extract_zp(zrow, b) : 0u, q);
        for (size_t ti = 0; ti < m_tail; ti++) {
          const size_t xb = (tt + ti) * Dz + bd;
          float a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0};
          for (int k = 0; k < 4; k++) {
            const int j = k * 8;
            for (int c = 0; c < 4; c++) {
              a0[c] = fmaf(load_x(x_f32, x, xb + j + c), q[j + c], a0[c]);
              a1[c] = fmaf(load_x(x_f32, x, xb + j + 4 + c), q[j + 4 + c], a1[c]);
            }
          }
          float cmb[4];
          for (int c = 0; c < 4; c++) cmb[c] = a0[c] + a1[c];
          const float blk = (cmb[0] + cmb[1]) + (cmb[2] + cmb[3]);
          const float prod = blk * scale;
          accs[ti] = accs[ti] + prod;
        }
      }
      const float bv = h2f(bias[n]);
      for (size_t ti = 0; ti < m_tail; ti++) store_out(out_f32, out, (tt + ti) * Nz + n, accs[ti] + bv);
    }
  }
}

/* ------------------------------------------------------------------ */
/* SwiGLU with clamp — :855-903                                        */
/* ------------------------------------------------------------------ */

void pfo_swiglu_clamp_f32(const float* gu, float* out, uint32_t T, uint32_t D) {
  const float LIMIT = 7.0f, ALPHA = 1.702f;
  for (size_t t = 0; t < T; t++) {
    const float* row = gu + t * 2 * (size_t)D;
    float* o = out + t * (size_t)D;
    size_t d = 0;
    for (; d + 4 <= D; d += 4) {
      for (int c = 0; c < 4; c++) {
        float gate = fminf(row[2 * (d + c)], LIMIT);
        float up = fmaxf(fminf(row[2 * (d + c) + 1], LIMIT), -LIMIT);
        float scaled = gate * ALPHA;
        float glu = gate * sigmoid_approx(scaled);
        o[d + c] = (up + 1.0f) * glu;
      }
    }
    for (; d < D; d++) {
      float gate = row[2 * d], up = row[2 * d + 1];
      if (gate > LIMIT) gate = LIMIT;
      if (up > LIMIT) up = LIMIT;
      if (up < -LIMIT) up = -LIMIT;
      float glu = gate * sigmoid_scalar(gate * ALPHA);
      o[d] = (up + 1.0f) * glu;
    }
  }
}

/* ------------------------------------------------------------------ */
/* softmax — :919-958                                                  */
/* ------------------------------------------------------------------ */

void pfo_softmax_f32(const float* x, float* out, uint32_t rows, uint32_t cols) {
  for (size_t r = 0; r < rows; r++) {
    const float* xr = x + r * cols;
    float* o = out + r * cols;
    float mx = xr[0];
    for (size_t c = 1; c < cols; c++) if (xr[c] > mx) mx = xr[c];
    float sum = 0.0f;
    for (size_t c = 0; c < cols; c++) { float e = expf(xr[c] - mx); o[c] = e; sum += e; }
    float inv = sum > 0.0f ? 1.0f / sum : 1.0f / (float)cols;
    for (size_t c = 0; c < cols; c++) o[c] *= inv;
  }
}

/* ------------------------------------------------------------------ */
/* elementwise — :969-1164                                             */
/* ------------------------------------------------------------------ */

void pfo_add_fp16(const uint16_t* a, const uint16_t* b, uint16_t* out, uint32_t n) {
  for (size_t i = 0; i < n; i++) out[i] = f2h(h2f(a[i]) + h2f(b[i]));
}

void pfo_gather_f32(const float* src, const int32_t* idx, float* dst, uint32_t m, uint32_t D) {
  for (size_t i = 0; i < m; i++) memcpy(dst + i * D, src + (size_t)idx[i] * D, sizeof(float) * D);
}

void pfo_scatter_add_weighted_f32(float* target, const float* values, const int32_t* idx, const float* weights,
                                  uint32_t m, uint32_t D) {
  for (size_t i = 0; i < m; i++) {
    float* tg = target + (size_t)idx[i] * D;
    const float* vr = values + i * D;
    const float w = weights[i];
    size_t d = 0;
    for (; d + 4 <= D; d += 4)
      for (int c = 0; c < 4; c++) tg[d + c] = fmaf(w, vr[d + c], tg[d + c]);
    for (; d < D; d++) tg[d] += w * vr[d];
  }
}

void pfo_cast_f32_to_fp16_scaled(const float* src, uint16_t* dst, uint32_t n, float scale) {
  for (size_t i = 0; i < n; i++) dst[i] = f2h(src[i] * scale);
}

/* ------------------------------------------------------------------ */
/* banded GQA attention with sinks — :1229-1432                        */
/* ------------------------------------------------------------------ */

/* dotBf16F32 (:1229-1262): 4 accumulators x 4 lanes over 16-element steps,
 * combined (a0+a1)+(a2+a3), lanes summed left to right, scalar tail. */
static inline float dot_f16(const uint16_t* a, const uint16_t* b, size_t n) {
  float acc[4][4] = {{0}};
  size_t i = 0;
  for (; i + 16 <= n; i += 16)
    for (int u = 0; u < 4; u++)
      for (int c = 0; c < 4; c++) acc[u][c] = fmaf(h2f(a[i + 4 * u + c]), h2f(b[i + 4 * u + c]), acc[u][c]);
  for (; i + 4 <= n; i += 4)
    for (int c = 0; c < 4; c++) acc[0][c] = fmaf(h2f(a[i + c]), h2f(b[i + c]), acc[0][c]);
  float cmb[4];
  for (int c = 0; c < 4; c++) cmb[c] = (acc[0][c] + acc[1][c]) + (acc[2][c] + acc[3][c]);
  float sum = cmb[0] + cmb[1] + cmb[2] + cmb[3];
  for (; i < n; i++) sum += h2f(a[i]) * h2f(b[i]);
  return sum;
}

void pfo_banded_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* sinks,
                          const uint8_t* mask, uint16_t* out, uint32_t T, uint32_t Hq, uint32_t Hkv,
                          uint32_t Dh, uint32_t W, uint32_t h0, uint32_t h1) {
  const size_t group = Hq / Hkv;
  const size_t qs = (size_t)Hq * Dh, ks = (size_t)Hkv * Dh;
  float* scores = (float*)malloc(sizeof(float) * (2 * (size_t)W + 2 + 8));
  float* acc = (float*)malloc(sizeof(float) * Dh);
  for (size_t tq = 0; tq < T; tq++) {
    for (size_t hq = h0; hq < h1; hq++) {
      const size_t hkv = hq / group;
      const size_t qb = tq * qs + hq * Dh;
      const size_t ws = tq > W ? tq - W : 0;
      const size_t we = tq + W + 1 < T ? tq + W + 1 : T;
      const size_t nk = we - ws;
      const float sink = sinks[hq];
      float mx = sink;
      for (size_t j = 0; j < nk; j++) {
        const size_t ak = ws + j;
        const int valid = mask ? (mask[ak] != 0) : 1;
        float s = valid ? dot_f16(q + qb, k + ak * ks + hkv * Dh, Dh) : -INFINITY;
        scores[j] = s;
        if (s > mx) mx = s;
      }
      scores[nk] = sink;
      const size_t total = nk + 1;
      float sv[4] = {0, 0, 0, 0};
      size_t i = 0;
      for (; i + 4 <= total; i += 4)
        for (int c = 0; c < 4; c++) { float e = exp_approx(scores[i + c] - mx); scores[i + c] = e; sv[c] += e; }
      float sum = sv[0] + sv[1] + sv[2] + sv[3];
      for (; i < total; i++) { float e = expf(scores[i] - mx); scores[i] = e; sum += e; }
      const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
      for (size_t d = 0; d < Dh; d++) acc[d] = 0.0f;
      for (size_t j = 0; j < nk; j++) {
        const float p = scores[j] * inv;
        const uint16_t* vr = v + (ws + j) * ks + hkv * Dh;
        size_t d = 0;
        for (; d + 4 <= Dh; d += 4)
          for (int c = 0; c < 4; c++) acc[d + c] = fmaf(p, h2f(vr[d + c]), acc[d + c]);
        for (; d < Dh; d++) acc[d] += p * h2f(vr[d]);
      }
      for (size_t d = 0; d < Dh; d++) out[qb + d] = f2h(acc[d]);
    }
  }
  free(scores);
  free(acc);
}

/* The reference's GPU-path attention, native/shaders/banded_attention.wgsl
 * (one 64-thread workgroup per (query, head)): scores by a sequential f32
 * fma over head_dim (:59-73), masked keys score NEG_INF = -1e30 (:56,72),
 * row max over the scores and the sink (:76-96), e = exp(s - max) with the
 * shader's exp (libm expf here; pass 2 :100-106), the sum as 64 strided
 * per-thread partials (the sink added to thread 0's) reduced by the shader's
 * tree (:110-126), inv = 1 / sum, p = e * inv (:131-137), then
 * out[d] = f16(sum_i fma(p_i, v_i[d], acc)) sequentially over the keys
 * (:141-151). fp16 values are widened IEEE-correctly (WGSL f32()) and the
 * output rounded RNE (WGSL f16()). */
static inline uint16_t f2h_ieee(float f) {
  const uint32_t x = f32_bits(f), sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);  /* NaN */
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  /* rounds to inf (>= 65520) */
  if (ax >= 0x38800000u) {                                    /* normal fp16: RNE */
    const uint32_t m = ax - 0x38000000u;
    return (uint16_t)(sign | ((m + 0x0fffu + ((m >> 13) & 1u)) >> 13));
  }
  return (uint16_t)(sign | (uint32_t)nearbyintf(bits_f32(ax) * 16777216.0f)); /* subnormal: RNE of f * 2^24 */
}

void pfo_f2h_ieee(const float* x, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = f2h_ieee(x[i]);
}

static inline float h2f_ieee(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ffu;
  if (e == 0) {
    const float v = ldexpf((float)m, -24);
    return sign ? -v : v;
  }
  if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

void pfo_banded_attention_wgsl(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* sinks,
                               const uint8_t* mask, uint16_t* out, uint32_t T, uint32_t Hq, uint32_t Hkv,
                               uint32_t Dh, uint32_t W) {
  const size_t group = Hq / Hkv;
  const size_t qs = (size_t)Hq * Dh, ks = (size_t)Hkv * Dh;
  const float NEG = -1e30f;
  float* scores = (float*)malloc(sizeof(float) * (2 * (size_t)W + 2));
  for (size_t tq = 0; tq < T; tq++) {
    for (size_t hq = 0; hq < Hq; hq++) {
      const size_t hkv = hq / group, qb = tq * qs + hq * Dh;
      const size_t ws = tq > W ? tq - W : 0;
      const size_t we = tq + W + 1 < T ? tq + W + 1 : T;
      const size_t nk = we - ws;
      float tmp[64];
      for (int t = 0; t < 64; t++) tmp[t] = NEG;
      for (size_t j = 0; j < nk; j++) {
        const size_t ak = ws + j;
        float s = NEG;
        if (!mask || mask[ak] != 0) {
          float dot = 0.0f;
          for (size_t d = 0; d < Dh; d++) dot = fmaf(h2f_ieee(q[qb + d]), h2f_ieee(k[ak * ks + hkv * Dh + d]), dot);
          s = dot;
        }
        scores[j] = s;
        if (s > tmp[j % 64]) tmp[j % 64] = s;
      }
      if (sinks[hq] > tmp[0]) tmp[0] = sinks[hq];
      for (int stride = 32; stride >= 1; stride /= 2)
        for (int t = 0; t < stride; t++) tmp[t] = fmaxf(tmp[t], tmp[t + stride]);
      const float row_max = tmp[0];
      for (int t = 0; t < 64; t++) tmp[t] = 0.0f;
      for (size_t j = 0; j < nk; j++) {
        const float e = expf(scores[j] - row_max);
        scores[j] = e;
        tmp[j % 64] = tmp[j % 64] + e;
      }
      tmp[0] = tmp[0] + expf(sinks[hq] - row_max);
      for (int stride = 32; stride >= 1; stride /= 2)
        for (int t = 0; t < stride; t++) tmp[t] = tmp[t] + tmp[t + stride];
      const float inv = tmp[0] > 0.0f ? 1.0f / tmp[0] : 0.0f;
      for (size_t j = 0; j < nk; j++) scores[j] = scores[j] * inv;
      for (size_t d = 0; d < Dh; d++) {
        float acc = 0.0f;
        for (size_t j = 0; j < nk; j++) acc = fmaf(scores[j], h2f_ieee(v[(ws + j) * ks + hkv * Dh + d]), acc);
        out[qb + d] = (uint16_t)f2h_ieee(acc);
      }
    }
  }
  free(scores);
}

/* ------------------------------------------------------------------ */
/* RoPE — :1460-1502 ; GatherBlockQuantized — :1523-1573               */
/* ------------------------------------------------------------------ */

void pfo_rope_apply(uint16_t* qk, const uint16_t* cs, const uint16_t* sn, uint32_t T, uint32_t H, uint32_t Dh) {
  const size_t half = Dh / 2;
  for (size_t t = 0; t < T; t++) {
    for (size_t h = 0; h < H; h++) {
      uint16_t* hb = qk + (t * H + h) * Dh;
      for (size_t p = 0; p < half; p++) {
        const float c = h2f(cs[t * half + p]), s = h2f(sn[t * half + p]);
        const float a = h2f(hb[2 * p]), b = h2f(hb[2 * p + 1]);
        const float ac = h2f(f2h(a * c)), bs = h2f(f2h(b * s));
        const float bc = h2f(f2h(b * c)), as_ = h2f(f2h(a * s));
        hb[2 * p] = f2h(ac - bs);
        hb[2 * p + 1] = f2h(bc + as_);
      }
    }
  }
}

void pfo_embed_lookup_int4(const uint8_t* ei, const uint16_t* es, const uint8_t* ez, const int32_t* ids,
                           uint16_t* out, uint32_t T, uint32_t V, uint32_t D) {
  const size_t nb = D / 32, is = D / 2, ss = nb, zs = (nb + 1) / 2;
  float q[32];
  for (size_t t = 0; t < T; t++) {
    const int32_t id = ids[t];
    uint16_t* o = out + t * D;
    if (id < 0 || (uint32_t)id >= V) { memset(o, 0, sizeof(uint16_t) * D); continue; }
    const size_t row = (size_t)id;
    for (size_t b = 0; b < nb; b++) {
      const float scale = h2f(es[row * ss + b]);
      decode_block(ei + row * is, b * 32, extract_zp(ez + row * zs, b), q);
      for (int j = 0; j < 32; j++) o[b * 32 + j] = f2h(q[j] * scale);
    }
  }
}

/* ------------------------------------------------------------------ */
/* YARN RoPE tables — browser/inference/rope.ts:27-144                 */
/* ------------------------------------------------------------------ */

/* rope.ts:82-108 f32ToFp16: the JS value is first stored to a Float32Array
 * (rounded to f32), zero short-circuits to +0, otherwise as zig/math.zig. */
static inline uint16_t js_f32_to_fp16(double f) {
  if (f == 0.0) return 0;
  return f2h((float)f);
}

void pfo_rope_tables(const pfo_config* cfg, uint32_t T, uint16_t* cos_t, uint16_t* sin_t) {
  const uint32_t hd = cfg->head_dim, half = hd / 2;
  const double theta = cfg->rope_theta, factor = cfg->rope_factor;
  float* extrap = (float*)malloc(sizeof(float) * half);
  float* interp = (float*)malloc(sizeof(float) * half);
  float* inv = (float*)malloc(sizeof(float) * half);
  for (uint32_t i = 0; i < half; i++) {
    double pos = pow(theta, (double)(2 * i) / (double)hd);
    extrap[i] = (float)(1.0 / pos);
    interp[i] = (float)(1.0 / (factor * pos));
  }
  const double PI = 3.141592653589793;
  double low = ((double)hd * log((double)cfg->rope_orig_max / (cfg->rope_beta_fast * 2.0 * PI))) / (2.0 * log(theta));
  double high = ((double)hd * log((double)cfg->rope_orig_max / (cfg->rope_beta_slow * 2.0 * PI))) / (2.0 * log(theta));
  if (cfg->rope_truncate) { low = floor(low); high = ceil(high); }
  if (low < 0) low = 0;
  if (high > (double)(hd - 1)) high = (double)(hd - 1);
  const double rmin = low, rmax = (high == low) ? low + 0.001 : high;
  for (uint32_t i = 0; i < half; i++) {
    double lin = ((double)i - rmin) / (rmax - rmin);
    double ramp = lin < 0 ? 0 : (lin > 1 ? 1 : lin);
    double ef = 1.0 - ramp;
    inv[i] = (float)((double)interp[i] * (1.0 - ef) + (double)extrap[i] * ef);
  }
  const double scaling = factor <= 1.0 ? 1.0 : 0.1 * log(factor) + 1.0;
  for (uint32_t t = 0; t < T; t++)
    for (uint32_t i = 0; i < half; i++) {
      double angle = (double)t * (double)inv[i];
      cos_t[(size_t)t * half + i] = js_f32_to_fp16(cos(angle) * scaling);
      sin_t[(size_t)t * half + i] = js_f32_to_fp16(sin(angle) * scaling);
    }
  free(extrap); free(interp); free(inv);
}

/* ------------------------------------------------------------------ */
/* thread helper for the MtPool partitioning (mt-pool.ts:421)          */
/* ------------------------------------------------------------------ */

typedef void (*slice_fn)(void* ctx, uint32_t start, uint32_t count, int worker);
typedef struct { slice_fn fn; void* ctx; uint32_t start, count; int worker; } slice_job;

static void* slice_entry(void* p) {
  slice_job* j = (slice_job*)p;
  j->fn(j->ctx, j->start, j->count, j->worker);
  return NULL;
}

/* Partition [0, total) as tStart = floor(w*total/n) (attention.ts:88-91)
 * and run each non-empty slice on its own thread. */
static void run_slices(slice_fn fn, void* ctx, uint32_t total, int n) {
  if (n <= 1) { fn(ctx, 0, total, 0); return; }
  pthread_t th[64];
  slice_job jobs[64];
  int started[64] = {0};
  for (int w = 0; w < n && w < 64; w++) {
    uint32_t s = (uint32_t)(((uint64_t)w * total) / (uint32_t)n);
    uint32_t e = (uint32_t)(((uint64_t)(w + 1) * total) / (uint32_t)n);
    jobs[w] = (slice_job){fn, ctx, s, e - s, w};
    if (e > s && pthread_create(&th[w], NULL, slice_entry, &jobs[w]) == 0) started[w] = 1;
    else if (e > s) slice_entry(&jobs[w]);
  }
  for (int w = 0; w < n && w < 64; w++) if (started[w]) pthread_join(th[w], NULL);
}

/* ------------------------------------------------------------------ */
/* router + expert dispatch — block.ts:49-102, expert.ts:104-212       */
/* ------------------------------------------------------------------ */

void pfo_router_select(const float* logits, int32_t* idx, float* weights, uint32_t T, uint32_t E, uint32_t K) {
  float* top = (float*)malloc(sizeof(float) * (size_t)T * K);
  pfo_topk_partial_f32(logits, idx, top, T, E, K);
  pfo_softmax_f32(top, weights, T, K);
  /* block.ts:99-101: JS multiplies by 1/K in double and stores to f32 */
  const double invK = 1.0 / (double)K;
  for (size_t i = 0; i < (size_t)T * K; i++) weights[i] = (float)((double)weights[i] * invK);
  free(top);
}

typedef struct {
  const pfo_config* cfg;
  const pfo_layer* layer;
  const float* hidden;
  const int32_t* ridx;
  const float* rw;
  float* acc;
  uint16_t* out;
} moe_ctx;

/* One expert-major pass over tokens [t0, t0+tc): expert.ts:125-211 for a
 * single slice, mt-expert.ts:95-180 when sliced. */
static void moe_slice(void* p, uint32_t t0, uint32_t tc, int worker) {
  (void)worker;
  moe_ctx* c = (moe_ctx*)p;
  const pfo_config* cfg = c->cfg;
  const uint32_t D = cfg->hidden, dff = cfg->dff, E = cfg->experts, K = cfg->topk;
  const size_t maxM = (size_t)tc * K;
  if (maxM == 0) return;
  int32_t* toks = (int32_t*)malloc(sizeof(int32_t) * maxM);
  float* wts = (float*)malloc(sizeof(float) * maxM);
  uint32_t* cnt = (uint32_t*)calloc(E + 1, sizeof(uint32_t));
  float* xg = (float*)malloc(sizeof(float) * maxM * D);
  float* gu = (float*)malloc(sizeof(float) * maxM * 2 * dff);
  float* glu = (float*)malloc(sizeof(float) * maxM * dff);
  float* of = (float*)malloc(sizeof(float) * maxM * D);
  /* count, then fill per expert in ascending (t, k) order */
  for (uint32_t t = t0; t < t0 + tc; t++)
    for (uint32_t k = 0; k < K; k++) {
      int32_t e = c->ridx[(size_t)t * K + k];
      if (e >= 0 && (uint32_t)e < E) cnt[e + 1]++;
    }
  for (uint32_t e = 0; e < E; e++) cnt[e + 1] += cnt[e];
  uint32_t* fill = (uint32_t*)malloc(sizeof(uint32_t) * E);
  memcpy(fill, cnt, sizeof(uint32_t) * E);
  for (uint32_t t = t0; t < t0 + tc; t++)
    for (uint32_t k = 0; k < K; k++) {
      int32_t e = c->ridx[(size_t)t * K + k];
      if (e < 0 || (uint32_t)e >= E) continue;
      toks[fill[e]] = (int32_t)t;
      wts[fill[e]] = c->rw[(size_t)t * K + k];
      fill[e]++;
    }
  const pfo_layer* L = c->layer;
  const size_t nbD = D / 32, nbF = dff / 32;
  for (uint32_t e = 0; e < E; e++) {
    const uint32_t m = cnt[e + 1] - cnt[e];
    if (m == 0) continue;
    const int32_t* ti = toks + cnt[e];
    const float* wi = wts + cnt[e];
    pfo_gather_f32(c->hidden, ti, xg, m, D);
    /* expertSlicePointers (expert.ts:62-80) */
    const size_t Ngu = 2 * (size_t)dff;
    pfo_matmul_int4block(1, 1, xg, L->gate_up.int4 + (size_t)e * Ngu * D / 2,
                         L->gate_up.scales + (size_t)e * Ngu * nbD,
                         L->gate_up.zp ? L->gate_up.zp + (size_t)e * Ngu * ((nbD + 1) / 2) : NULL,
                         L->gate_up.bias + (size_t)e * Ngu, gu, m, (uint32_t)Ngu, D);
    pfo_swiglu_clamp_f32(gu, glu, m, dff);
    pfo_matmul_int4block(1, 1, glu, L->down.int4 + (size_t)e * D * dff / 2,
                         L->down.scales + (size_t)e * D * nbF,
                         L->down.zp ? L->down.zp + (size_t)e * D * ((nbF + 1) / 2) : NULL,
                         L->down.bias + (size_t)e * D, of, m, D, dff);
    pfo_scatter_add_weighted_f32(c->acc, of, ti, wi, m, D);
  }
  /* final = fp16(acc * K), per slice (mt-expert.ts:182-188) */
  pfo_cast_f32_to_fp16_scaled(c->acc + (size_t)t0 * D, c->out + (size_t)t0 * D, tc * D, (float)K);
  free(toks); free(wts); free(cnt); free(fill); free(xg); free(gu); free(glu); free(of);
}

int pfo_expert_dispatch(const pfo_config* cfg, const pfo_layer* layer, const float* hidden_f32,
                        const int32_t* routing_idx, const float* routing_w, uint16_t* out, uint32_t T,
                        int n_slices) {
  float* acc = (float*)calloc((size_t)T * cfg->hidden, sizeof(float));
  if (!acc) return -1;
  moe_ctx c = {cfg, layer, hidden_f32, routing_idx, routing_w, acc, out};
  run_slices(moe_slice, &c, T, n_slices < 1 ? 1 : n_slices);
  free(acc);
  return 0;
}

/* ------------------------------------------------------------------ */
/* attention + block + model — attention.ts, block.ts, model.ts        */
/* ------------------------------------------------------------------ */

typedef struct {
  const pfo_config* cfg;
  const pfo_layer* L;
  const float* x;          /* hidden f32 [T, D] */
  uint16_t *q, *k, *v;
  const uint16_t *cos_t, *sin_t;
} qkv_ctx;

/* attention.ts:94-121: per T slice, Q/K/V matmuls then RoPE. */
static void qkv_slice(void* p, uint32_t t0, uint32_t tc, int w) {
  (void)w;
  qkv_ctx* c = (qkv_ctx*)p;
  const pfo_config* cfg = c->cfg;
  const uint32_t D = cfg->hidden, Hq = cfg->heads, Hkv = cfg->kv_heads, hd = cfg->head_dim;
  const float* x = c->x + (size_t)t0 * D;
  uint16_t* q = c->q + (size_t)t0 * Hq * hd;
  uint16_t* k = c->k + (size_t)t0 * Hkv * hd;
  uint16_t* v = c->v + (size_t)t0 * Hkv * hd;
  pfo_matmul_int4block(1, 0, x, c->L->q.int4, c->L->q.scales, c->L->q.zp, c->L->q.bias, q, tc, Hq * hd, D);
  pfo_matmul_int4block(1, 0, x, c->L->k.int4, c->L->k.scales, c->L->k.zp, c->L->k.bias, k, tc, Hkv * hd, D);
  pfo_matmul_int4block(1, 0, x, c->L->v.int4, c->L->v.scales, c->L->v.zp, c->L->v.bias, v, tc, Hkv * hd, D);
  const size_t off = (size_t)t0 * (hd / 2);
  pfo_rope_apply(q, c->cos_t + off, c->sin_t + off, tc, Hq, hd);
  pfo_rope_apply(k, c->cos_t + off, c->sin_t + off, tc, Hkv, hd);
}

typedef struct {
  const pfo_config* cfg;
  const pfo_layer* L;
  const uint16_t *q, *k, *v;
  const uint8_t* mask;
  uint16_t* out;
  uint32_t T;
} att_ctx;

static void att_slice(void* p, uint32_t h0, uint32_t hc, int w) {
  (void)w;
  att_ctx* c = (att_ctx*)p;
  pfo_banded_attention(c->q, c->k, c->v, c->L->sinks, c->mask, c->out, c->T, c->cfg->heads, c->cfg->kv_heads,
                       c->cfg->head_dim, c->cfg->window, h0, h0 + hc);
}

typedef struct {
  int x_f32, out_f32;
  const void* x;
  const pfo_qweight* w;
  void* out;
  uint32_t N, D;
  size_t x_es, out_es;      /* element sizes */
} mm_ctx;

static void mm_slice(void* p, uint32_t t0, uint32_t tc, int w) {
  (void)w;
  mm_ctx* c = (mm_ctx*)p;
  pfo_matmul_int4block(c->x_f32, c->out_f32, (const char*)c->x + (size_t)t0 * c->D * c->x_es, c->w->int4,
                       c->w->scales, c->w->zp, c->w->bias, (char*)c->out + (size_t)t0 * c->N * c->out_es, tc,
                       c->N, c->D);
}

typedef struct {
  const uint16_t *a, *b, *g;
  uint16_t* sum;
  float* norm;
  uint32_t D;
  float eps;
} arn_ctx;

static void arn_slice(void* p, uint32_t t0, uint32_t tc, int w) {
  (void)w;
  arn_ctx* c = (arn_ctx*)p;
  const size_t o = (size_t)t0 * c->D;
  pfo_add_rmsnorm_fp16_to_f32(c->a + o, c->b + o, c->g, c->sum + o, c->norm + o, tc, c->D, c->eps);
}

/* ridx_out (optional, [T][K]): the layer's routed expert ids */
static int block_forward_impl(const pfo_config* cfg, const pfo_layer* L, const uint16_t* input, uint16_t* output,
                              const uint16_t* cos_t, const uint16_t* sin_t, const uint8_t* mask, uint32_t T,
                              int n_threads, int32_t* ridx_out) {
  const uint32_t D = cfg->hidden, Hq = cfg->heads, Hkv = cfg->kv_heads, hd = cfg->head_dim;
  const uint32_t E = cfg->experts, K = cfg->topk;
  const int N = n_threads < 1 ? 1 : n_threads;
  /* MtPool thresholds: T-partition only when T >= 2N (attention.ts:87),
   * H_q partition when Hq >= 2N (:156). */
  const int nT = (N > 1 && T >= (uint32_t)(2 * N)) ? N : 1;
  const int nH = (N > 1 && Hq >= (uint32_t)(2 * N)) ? N : 1;
  float* hf = (float*)malloc(sizeof(float) * (size_t)T * D);
  uint16_t* q = (uint16_t*)malloc(2 * (size_t)T * Hq * hd);
  uint16_t* k = (uint16_t*)malloc(2 * (size_t)T * Hkv * hd);
  uint16_t* v = (uint16_t*)malloc(2 * (size_t)T * Hkv * hd);
  uint16_t* ao = (uint16_t*)malloc(2 * (size_t)T * Hq * hd);
  float* af = (float*)malloc(sizeof(float) * (size_t)T * Hq * hd);
  uint16_t* attn = (uint16_t*)malloc(2 * (size_t)T * D);
  uint16_t* res2 = (uint16_t*)malloc(2 * (size_t)T * D);
  float* n2 = (float*)malloc(sizeof(float) * (size_t)T * D);
  float* rl = (float*)malloc(sizeof(float) * (size_t)T * E);
  int32_t* ridx = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * K);
  float* rw = (float*)malloc(sizeof(float) * (size_t)T * K);
  uint16_t* moe = (uint16_t*)malloc(2 * (size_t)T * D);
  int rc = -1;
  if (!hf || !q || !k || !v || !ao || !af || !attn || !res2 || !n2 || !rl || !ridx || !rw || !moe) goto done;

  /* block.ts:124-129 (single call, not partitioned) */
  pfo_rms_norm_fp16_to_f32(input, L->input_ln, hf, T, D, cfg->eps);
  /* attention.ts:74-148 */
  {
    qkv_ctx c = {cfg, L, hf, q, k, v, cos_t, sin_t};
    run_slices(qkv_slice, &c, T, nT);
  }
  {
    att_ctx c = {cfg, L, q, k, v, mask, ao, T};
    run_slices(att_slice, &c, Hq, nH);
  }
  pfo_fp16_to_f32_n(ao, af, (size_t)T * Hq * hd);
  {
    mm_ctx c = {1, 0, af, &L->o, attn, D, Hq * hd, 4, 2};
    run_slices(mm_slice, &c, T, nT);
  }
  /* block.ts:140-173 */
  {
    arn_ctx c = {input, attn, L->post_ln, res2, n2, D, cfg->eps};
    run_slices(arn_slice, &c, T, nT);
  }
  /* routerForward (block.ts:61-101) */
  {
    mm_ctx c = {1, 1, n2, &L->router, rl, E, D, 4, 4};
    run_slices(mm_slice, &c, T, nT);
  }
  pfo_router_select(rl, ridx, rw, T, E, K);
  if (ridx_out) memcpy(ridx_out, ridx, sizeof(int32_t) * (size_t)T * K);
  /* expertDispatch: MT mode always takes the sliced path (expert.ts:115-121) */
  if (pfo_expert_dispatch(cfg, L, n2, ridx, rw, moe, T, N) != 0) goto done;
  pfo_add_fp16(res2, moe, output, T * D);
  rc = 0;
done:
  free(hf); free(q); free(k); free(v); free(ao); free(af); free(attn); free(res2); free(n2);
  free(rl); free(ridx); free(rw); free(moe);
  return rc;
}

int pfo_block_forward(const pfo_config* cfg, const pfo_layer* L, const uint16_t* input, uint16_t* output,
                      const uint16_t* cos_t, const uint16_t* sin_t, const uint8_t* mask, uint32_t T,
                      int n_threads) {
  return block_forward_impl(cfg, L, input, output, cos_t, sin_t, mask, T, n_threads, NULL);
}

int pfo_model_forward_route(const pfo_config* cfg, const pfo_model* m, const int32_t* ids, const uint8_t* mask,
                            uint32_t T, int n_threads, uint16_t* logits, int32_t* ridx_out) {
  const uint32_t D = cfg->hidden, half = cfg->head_dim / 2;
  uint16_t* cs = (uint16_t*)malloc(2 * (size_t)T * half);
  uint16_t* sn = (uint16_t*)malloc(2 * (size_t)T * half);
  uint16_t* h0 = (uint16_t*)malloc(2 * (size_t)T * D);
  uint16_t* h1 = (uint16_t*)malloc(2 * (size_t)T * D);
  float* cx = (float*)malloc(sizeof(float) * (size_t)T * D);
  int rc = -1;
  if (!cs || !sn || !h0 || !h1 || !cx) goto done;
  /* wasm.ts:753-764: an all-ones mask is elided */
  const uint8_t* mk = NULL;
  if (mask)
    for (uint32_t i = 0; i < T; i++) if (mask[i] != 1) { mk = mask; break; }
  pfo_rope_tables(cfg, T, cs, sn);
  pfo_embed_lookup_int4(m->embed_int4, m->embed_scales, m->embed_zp, ids, h0, T, cfg->vocab, D);
  uint16_t *src = h0, *dst = h1;
  for (uint32_t l = 0; l < cfg->layers; l++) {
    if (block_forward_impl(cfg, &m->layers[l], src, dst, cs, sn, mk, T, n_threads,
                           ridx_out ? ridx_out + (size_t)l * T * cfg->topk : NULL) != 0) goto done;
    uint16_t* t = src; src = dst; dst = t;
  }
  pfo_rms_norm_fp16_to_f32(src, m->final_ln, cx, T, D, cfg->eps);
  pfo_matmul_int4block(1, 0, cx, m->score.int4, m->score.scales, m->score.zp, m->score.bias, logits, T,
                       cfg->classes, D);
  rc = 0;
done:
  free(cs); free(sn); free(h0); free(h1); free(cx);
  return rc;
}

int pfo_model_forward(const pfo_config* cfg, const pfo_model* m, const int32_t* ids, const uint8_t* mask,
                      uint32_t T, int n_threads, uint16_t* logits) {
  return pfo_model_forward_route(cfg, m, ids, mask, T, n_threads, logits, NULL);
}
