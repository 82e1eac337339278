// kernels_misc.hip — HBM-bound kernels of the forward: the
// GatherBlockQuantized embedding, RMSNorm variants, element-wise ops, the
// router top-k, the MoE routing plan (a deterministic counting sort) and the
// MoE combine. Reference semantics: packages/textsift/src/zig/wasm_exports.zig
// (line ranges cited per kernel).
#include "common.h"
#include "epilogue.h"
#include "pfhip_internal.h"
#include "topk.h"
#include "combine.h"

namespace pf {

namespace {

constexpr int ROWS_PER_BLOCK = 4;  // one wave per row, 4 waves per block

// ----------------------------------------------------------------------------
// GatherBlockQuantized (embed_lookup_int4, :1523-1573). A thread takes one
// dword of packed nibbles (8 output values, 16 bytes out) at the same
// position u of EMB_TOK rows: it issues every id load, then every table
// load, then converts and stores, so a wave has that many independent
// memory chains in flight and the grid is a few rounds of waves. Consecutive
// threads take consecutive dwords of a row: every wave's stores of one row
// form a contiguous block, and the 4 threads of a quant block read its scale
// and zero-point from one line. fp16((q - zp) * scale) is a single rounding of
// an exact product, so the output is bit-identical to the reference. Ids
// outside [0, V) give a zero row.
// NT: non-temporal stores (the stand-alone op: 15.6 -> 13.1 us warm, 18.2 ->
// 14.4 us cold at 32768 x 640; in the forward they would cost the RMSNorm
// that reads the rows next its cache hits, +3 us).
constexpr int EMB_TOK = 4;  // measured: 2, 4 and 8 within 5 %, 16 slower
template <bool NT>
__global__ __launch_bounds__(256) void k_embed(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                               const uint8_t* __restrict__ zp, const int32_t* __restrict__ ids,
                                               uint16_t* __restrict__ out, int T, int V, int D) {
  const int nd = D >> 3, nb = D >> 5;
  // 32-bit index arithmetic (the launcher checks groups * nd < 2^31): a
  // 64-bit division is a long instruction sequence
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  const int groups = (T + EMB_TOK - 1) / EMB_TOK;
  if (i >= (uint32_t)groups * (uint32_t)nd) return;
  const int g = (int)(i / (uint32_t)nd), u = (int)(i % (uint32_t)nd);
  const int blk = u >> 2;
  int id[EMB_TOK];
#pragma unroll
  for (int r = 0; r < EMB_TOK; ++r) {
    const int t = min(g * EMB_TOK + r, T - 1);
    id[r] = ids[t];
  }
  uint32_t w[EMB_TOK];
  uint16_t sb[EMB_TOK];
  uint8_t zb[EMB_TOK];
#pragma unroll
  for (int r = 0; r < EMB_TOK; ++r) {
    const size_t row = (id[r] >= 0 && id[r] < V) ? (size_t)id[r] : 0;  // out-of-range ids read row 0, stored as 0
    w[r] = reinterpret_cast<const uint32_t*>(q + row * (D >> 1))[u];
    sb[r] = s[row * nb + blk];
    zb[r] = zp[row * ((nb + 1) >> 1) + (blk >> 1)];
  }
#pragma unroll
  for (int r = 0; r < EMB_TOK; ++r) {
    const int t = g * EMB_TOK + r;
    if (t >= T) break;
    u4_t res = {0u, 0u, 0u, 0u};
    if (id[r] >= 0 && id[r] < V) {
      const float sc = wasm_h2f(sb[r]);
      const int z = (blk & 1) ? (zb[r] >> 4) : (zb[r] & 0xF);
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (float)((int)((w[r] >> (4 * j)) & 0xFu) - z) * sc;
      const u2_t a = to_f16x4_z(v), c = to_f16x4_z(v + 4);
      res = u4_t{a.x, a.y, c.x, c.y};
    }
    u4_t* dst = reinterpret_cast<u4_t*>(out + (size_t)t * D) + u;
    if constexpr (NT) __builtin_nontemporal_store(res, dst);
    else *dst = res;
  }
}

// ----------------------------------------------------------------------------
// RMSNorm family (:186-350). One wave per row; lane l holds elements
// 4l + 256j .. +3 (8-byte loads), so D must be a multiple of 4 and <= 1024.
// Widening is the reference's bit trick (wasm_h2f).
constexpr int MAXJ = 4;  // 256-element slices per row


template <int MODE>
__global__ __launch_bounds__(256) void k_rms_norm(const uint16_t* __restrict__ x, const uint16_t* __restrict__ g,
                                                  void* __restrict__ out, uint16_t* __restrict__ out_lo, int T, int D,
                                                  float eps) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (t >= T) return;
  const size_t base = (size_t)t * D;
  float v[MAXJ][4];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const int d = 4 * lane + 256 * j;
    if (d < D) {
      h4_to_f(*reinterpret_cast<const u2_t*>(x + base + d), v[j]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) v[j][r] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) ss += v[j][r] * v[j][r];
  }
  ss = wave_sum(ss);
  const float inv_rms = 1.0f / sqrtf(ss * (1.0f / (float)D) + eps);
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const int d = 4 * lane + 256 * j;
    if (d < D) {
      float gm[4], y[4];
      h4_to_f(*reinterpret_cast<const u2_t*>(g + d), gm);
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = v[j][r] * inv_rms * gm[r];
      put4<MODE>(out, out_lo, base + d, y);
    }
  }
}

// rms_norm with fp16 output for D = 128 NU: one wave takes 4 rows as 4 D / 8
// = 64 NU 16-byte units, NU per lane (unit u = 64 i + lane of the wave's
// rows; row u / (D / 8)), so every load and store instruction of the wave
// moves 1 KB with all lanes active (the 8-byte, one-row-per-wave form moved
// 512 B, the last instruction of a 640-wide row half empty). Each lane keeps
// a partial sum of squares per row; the 4 row sums are wave reductions.
template <int NU>
__global__ __launch_bounds__(256) void k_rms_norm4(const uint16_t* __restrict__ x, const uint16_t* __restrict__ g,
                                                   uint16_t* __restrict__ out, int T, float eps) {
  constexpr int D = 128 * NU, UPR = D / 8;
  const int lane = threadIdx.x & 63;
  const int t0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 4;
  if (t0 >= T) return;
  u4_t raw[NU];
  int row[NU], col[NU];
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int u = 64 * i + lane;
    row[i] = u / UPR;
    col[i] = (u - row[i] * UPR) * 8;
    const int t = min(t0 + row[i], T - 1);
    raw[i] = *reinterpret_cast<const u4_t*>(x + (size_t)t * D + col[i]);
  }
  float v[NU][8];
  float ss[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    h4_to_f(u2_t{raw[i].x, raw[i].y}, v[i]);
    h4_to_f(u2_t{raw[i].z, raw[i].w}, v[i] + 4);
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < 8; ++r) s += v[i][r] * v[i][r];
#pragma unroll
    for (int r = 0; r < 4; ++r) ss[r] += row[i] == r ? s : 0.0f;
  }
  float inv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) inv[r] = 1.0f / sqrtf(wave_sum(ss[r]) * (1.0f / (float)D) + eps);
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int t = t0 + row[i];
    const float ir = row[i] == 0 ? inv[0] : row[i] == 1 ? inv[1] : row[i] == 2 ? inv[2] : inv[3];
    const u4_t gw = *reinterpret_cast<const u4_t*>(g + col[i]);
    float gm[8], y[8];
    h4_to_f(u2_t{gw.x, gw.y}, gm);
    h4_to_f(u2_t{gw.z, gw.w}, gm + 4);
#pragma unroll
    for (int r = 0; r < 8; ++r) y[r] = v[i][r] * ir * gm[r];
    // (the zero-tolerant fast test: the embedding rows this norm follows hold
    // exact zeros wherever q == zp, which the plain test sends to the exact
    // software path -- two fifths of the units of the forward's synthetic
    // model, most of this kernel's time)
    const u2_t lo = to_f16x4_z(y), hi = to_f16x4_z(y + 4);
    if (t < T) *reinterpret_cast<u4_t*>(out + (size_t)t * D + col[i]) = u4_t{lo.x, lo.y, hi.x, hi.y};
  }
}

// The embedding gather and the model's first RMSNorm in one pass (fp16
// numerics, D = 128 NU): embed_lookup_int4 (zig/wasm_exports.zig:1523-1573)
// then rms_norm (:186-218). The units are k_rms_norm4's (a wave takes 4 rows,
// lane l the 16-byte units u = 64 i + l, row u / (D / 8)), and a unit is
// exactly what one k_embed thread makes of one dword of a table row: 8
// nibbles -> fp16((q - zp) * scale). Each lane stores its embedded units (the
// residual stream), widens them as k_rms_norm4 widens what it loads and
// normalises them in k_rms_norm4's order, so both outputs are the bits of the
// two-kernel form, without the embedded rows' write-then-read in between.
// Ids outside [0, V) give a zero row (and a zero-row norm).
template <int NU>
__global__ __launch_bounds__(256) void k_embed_rms_norm4(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                                         const uint8_t* __restrict__ zp,
                                                         const int32_t* __restrict__ ids,
                                                         const uint16_t* __restrict__ g, uint16_t* __restrict__ h,
                                                         uint16_t* __restrict__ out, int T, int V, float eps) {
  constexpr int D = 128 * NU, UPR = D / 8, NB = D / 32, NZ = (NB + 1) / 2;
  const int lane = threadIdx.x & 63;
  const int t0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 4;
  if (t0 >= T) return;
  int id[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) id[r] = ids[min(t0 + r, T - 1)];
  uint32_t w[NU];
  uint16_t sb[NU];
  uint8_t zb[NU];
  int row[NU], dw[NU];
  bool ok[NU];
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int u = 64 * i + lane;
    row[i] = u / UPR;
    dw[i] = u - row[i] * UPR;  // the dword of the table row (8 values)
    const int idr = row[i] == 0 ? id[0] : row[i] == 1 ? id[1] : row[i] == 2 ? id[2] : id[3];
    ok[i] = idr >= 0 && idr < V;
    const uint32_t rr = ok[i] ? (uint32_t)idr : 0u;  // out-of-range ids read row 0, stored as 0
    w[i] = reinterpret_cast<const uint32_t*>(q + (size_t)rr * (D / 2))[dw[i]];
    sb[i] = s[(size_t)rr * NB + (dw[i] >> 2)];
    zb[i] = zp[(size_t)rr * NZ + (dw[i] >> 3)];
  }
  float v[NU][8];
  float ss[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    u4_t res = {0u, 0u, 0u, 0u};
    if (ok[i]) {
      const float sc = wasm_h2f(sb[i]);
      const int z = ((dw[i] >> 2) & 1) ? (zb[i] >> 4) : (zb[i] & 0xF);
      float e[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) e[j] = (float)((int)((w[i] >> (4 * j)) & 0xFu) - z) * sc;
      const u2_t a = to_f16x4_z(e), c = to_f16x4_z(e + 4);
      res = u4_t{a.x, a.y, c.x, c.y};
    }
    const int t = t0 + row[i];
    if (t < T) *reinterpret_cast<u4_t*>(h + (size_t)t * D + dw[i] * 8) = res;
    h4_to_f(u2_t{res.x, res.y}, v[i]);
    h4_to_f(u2_t{res.z, res.w}, v[i] + 4);
    float sq = 0.0f;
#pragma unroll
    for (int r = 0; r < 8; ++r) sq += v[i][r] * v[i][r];
#pragma unroll
    for (int r = 0; r < 4; ++r) ss[r] += row[i] == r ? sq : 0.0f;
  }
  float inv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) inv[r] = 1.0f / sqrtf(wave_sum(ss[r]) * (1.0f / (float)D) + eps);
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int t = t0 + row[i];
    const float ir = row[i] == 0 ? inv[0] : row[i] == 1 ? inv[1] : row[i] == 2 ? inv[2] : inv[3];
    const u4_t gw = *reinterpret_cast<const u4_t*>(g + dw[i] * 8);
    float gm[8], y[8];
    h4_to_f(u2_t{gw.x, gw.y}, gm);
    h4_to_f(u2_t{gw.z, gw.w}, gm + 4);
#pragma unroll
    for (int r = 0; r < 8; ++r) y[r] = v[i][r] * ir * gm[r];
    const u2_t lo = to_f16x4_z(y), hi = to_f16x4_z(y + 4);
    if (t < T) *reinterpret_cast<u4_t*>(out + (size_t)t * D + dw[i] * 8) = u4_t{lo.x, lo.y, hi.x, hi.y};
  }
}

// add_rmsnorm_fp16_to_f32 (:288-350): sum = a + b (fp16 store), sumsq of the
// unrounded f32 sum, normalise the rounded sum.
template <int MODE>
__global__ __launch_bounds__(256) void k_add_rms_norm(const uint16_t* __restrict__ a,
                                                      const uint16_t* __restrict__ bb,
                                                      const uint16_t* __restrict__ g, uint16_t* __restrict__ sum_out,
                                                      void* __restrict__ norm_out, uint16_t* __restrict__ norm_lo,
                                                      int T, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (t >= T) return;
  const size_t base = (size_t)t * D;
  u2_t hs[MAXJ];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const int d = 4 * lane + 256 * j;
    hs[j] = u2_t{0u, 0u};
    if (d < D) {
      float av[4], bv[4], sv[4];
      h4_to_f(*reinterpret_cast<const u2_t*>(a + base + d), av);
      h4_to_f(*reinterpret_cast<const u2_t*>(bb + base + d), bv);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[r] = av[r] + bv[r];
        ss += sv[r] * sv[r];
      }
      hs[j] = to_f16x4(sv);
      *reinterpret_cast<u2_t*>(sum_out + base + d) = hs[j];
    }
  }
  ss = wave_sum(ss);
  const float inv_rms = 1.0f / sqrtf(ss * (1.0f / (float)D) + eps);
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const int d = 4 * lane + 256 * j;
    if (d < D) {
      float hv[4], gm[4], y[4];
      h4_to_f(hs[j], hv);
      h4_to_f(*reinterpret_cast<const u2_t*>(g + d), gm);
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = hv[r] * inv_rms * gm[r];
      put4<MODE>(norm_out, norm_lo, base + d, y);
    }
  }
}

// ----------------------------------------------------------------------------
// Element-wise (:969-1164).
__global__ void k_split_f32(const float* x, uint16_t* hi, uint16_t* lo, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    split_hilo(x[i], hi[i], lo[i]);
}
__global__ void k_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* o, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    o[i] = wasm_f2h(wasm_h2f(a[i]) + wasm_h2f(b[i]));
}
__global__ void k_cast_f16_f32(const uint16_t* s, float* d, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    d[i] = wasm_h2f(s[i]);
}
__global__ void k_cast_f16_f32_ieee(const uint16_t* s, float* d, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    d[i] = hw_h2f(s[i]);
}
__global__ void k_cast_f32_f16_scaled(const float* s, uint16_t* d, size_t n, float scale) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    d[i] = wasm_f2h(s[i] * scale);
}
__global__ void k_zero_f32(float* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0.0f;
}
// swiglu_clamp_f32 (:855-903): the vector path (polynomial sigmoid) for the
// D & ~3 leading columns, the scalar path (libm exp) for the tail.
__global__ void k_swiglu(const float* gu, float* out, int rows, int dff) {
  const size_t n = (size_t)rows * dff;
  const int vec_end = dff & ~3;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = i / dff;
    const int d = (int)(i % dff);
    const float gr = gu[r * 2 * dff + 2 * d], ur = gu[r * 2 * dff + 2 * d + 1];
    if (d < vec_end) {
      out[i] = swiglu_clamp(gr, ur);
    } else {
      float gate = fminf(gr, 7.0f), up = fmaxf(fminf(ur, 7.0f), -7.0f);
      const float x = gate * 1.702f;
      const float sg = x >= 0.0f ? 1.0f / (1.0f + expf(-x)) : expf(x) / (1.0f + expf(x));
      out[i] = (up + 1.0f) * (gate * sg);
    }
  }
}
// rope_apply (:1460-1502): rows of `row_stride` halves, H heads of hd.
__global__ void k_rope(uint16_t* qk, const uint16_t* cs, const uint16_t* sn, int T, int H, int hd, int row_stride,
                       int seq_len) {
  const int half = hd >> 1;
  const size_t n = (size_t)T * H * half;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int p = (int)(i % half);
    const size_t th = i / half;
    const int h = (int)(th % H);
    const size_t t = th / H;
    const int pos = (int)(t % (size_t)seq_len);
    uint16_t* hb = qk + t * row_stride + (size_t)h * hd;
    const float c = wasm_h2f(cs[(size_t)pos * half + p]), s = wasm_h2f(sn[(size_t)pos * half + p]);
    const float a = wasm_h2f(hb[2 * p]), b = wasm_h2f(hb[2 * p + 1]);
    const float ac = wasm_h2f(wasm_f2h(a * c)), bs = wasm_h2f(wasm_f2h(b * s));
    const float bc = wasm_h2f(wasm_f2h(b * c)), as_ = wasm_h2f(wasm_f2h(a * s));
    hb[2 * p] = wasm_f2h(ac - bs);
    hb[2 * p + 1] = wasm_f2h(bc + as_);
  }
}

// ----------------------------------------------------------------------------
// Router top-k + softmax (topk_partial_f32 :367-426, softmax_f32 :919-958;
// the insertion order and the weights are in topk.h): output sorted by
// logit descending, ties keep the lower expert id first.
constexpr int MAXK = 8;
// One wave per token; lane l holds logits l, l+64, l+128, l+192. Without
// NaNs the insertion top-k equals K rounds of "largest value, lowest index
// among equal values", done as wave reductions; a row with a NaN takes the
// sequential insertion path (whose comparisons NaN short-circuits).
constexpr int TOPK_PL = 4;  // E <= 256
template <int K>
__global__ __launch_bounds__(256) void k_router_topk(const float* __restrict__ logits, int32_t* __restrict__ idx,
                                                     float* __restrict__ w, int T, int E, float wscale) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* x = logits + (size_t)t * E;
  float xv[TOPK_PL];
  bool live[TOPK_PL];
  bool nan = false;
#pragma unroll
  for (int j = 0; j < TOPK_PL; ++j) {
    const int c = lane + 64 * j;
    live[j] = c < E;
    xv[j] = live[j] ? x[c] : -INFINITY;
    nan = nan || (live[j] && xv[j] != xv[j]);
  }
  float V[K];
  int I[K];
  if (__any(nan)) {
    if (lane == 0) topk_insertion<K>([&](int c) { return x[c]; }, E, V, I);
    // broadcast lane 0's result
#pragma unroll
    for (int k = 0; k < K; ++k) {
      V[k] = __shfl(V[k], 0, 64);
      I[k] = __shfl(I[k], 0, 64);
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < TOPK_PL; ++j) {
        const int c = lane + 64 * j;
        const bool take = live[j] & ((xv[j] > bv) | ((xv[j] == bv) & (c < bi)));
        bv = take ? xv[j] : bv;
        bi = take ? c : bi;
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        const bool take = (ov > bv) | ((ov == bv) & (oi < bi));
        bv = take ? ov : bv;
        bi = take ? oi : bi;
      }
      V[k] = bv;
      I[k] = bi;
#pragma unroll
      for (int j = 0; j < TOPK_PL; ++j) live[j] = live[j] & (lane + 64 * j != bi);
    }
  }
  if (lane == 0) topk_write<K>(V, I, wscale, idx + (size_t)t * K, w + (size_t)t * K);
}

// ----------------------------------------------------------------------------
// MoE routing plan: a stable counting sort of the T*K (token, k) pairs by
// expert, reproducing the reference's per-expert lists (for e ascending, the
// pairs with expert e in ascending token order: browser/inference/
// expert.ts:125-145). Deterministic: no atomics anywhere.
constexpr int RBLK = 1024;          // tokens per counting block
constexpr int BWS = RBLK / 32 + 1;  // bitmap words per expert in LDS (padded: rows in distinct banks)

// Per-block expert bitmaps: bit t of bits[e][t / 32] is set when token t of
// the block routes to expert e. OR is order-independent, so the bitmap (and
// everything derived from it) is deterministic. Entries with an expert id
// outside [0, E) are ignored.
// This thread's token's K expert ids (token t0 + threadIdx.x; -1 past the
// block's nt tokens and past K), loaded once and kept in registers.
__device__ __forceinline__ void moe_load_ids(const int32_t* __restrict__ idx, int t0, int nt, int K, int (&ids)[MAXK]) {
  const int tl = threadIdx.x;
#pragma unroll
  for (int k = 0; k < MAXK; ++k) ids[k] = (k < K && tl < nt) ? idx[(size_t)(t0 + tl) * K + k] : -1;
}

__device__ __forceinline__ void moe_block_bitmap_ids(const int (&ids)[MAXK], uint32_t* bits, int E) {
  for (int i = threadIdx.x; i < E * BWS; i += blockDim.x) bits[i] = 0u;
  __syncthreads();
  const int tl = threadIdx.x;
#pragma unroll
  for (int k = 0; k < MAXK; ++k) {
    const int e = ids[k];
    if ((unsigned)e < (unsigned)E) atomicOr(&bits[e * BWS + (tl >> 5)], 1u << (tl & 31));
  }
  __syncthreads();
}

__device__ __forceinline__ void moe_block_bitmap(const int32_t* __restrict__ idx, uint32_t* bits, int t0, int nt,
                                                 int K, int E) {
  int ids[MAXK];
  moe_load_ids(idx, t0, nt, K, ids);
  moe_block_bitmap_ids(ids, bits, E);
}

// pre[e][w] = tokens of the block routed to e among words 0 .. w-1 of the
// bitmap (so a token's rank is pre[e][w] plus a popcount within its word)
__device__ __forceinline__ void moe_word_prefix(const uint32_t* bits, uint16_t* pre, int E) {
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    uint32_t w[RBLK / 32];
#pragma unroll
    for (int u = 0; u < RBLK / 32; ++u) w[u] = bits[e * BWS + u];
    int run = 0;
#pragma unroll
    for (int u = 0; u < RBLK / 32; ++u) {
      pre[e * BWS + u] = (uint16_t)run;
      run += __popc(w[u]);
    }
  }
  __syncthreads();
}

// The grouped-GEMM tile list (expert, row0, rows), written by all threads of
// the workgroup: tile ti belongs to the last expert whose first tile (tile0,
// an exclusive prefix over experts) is <= ti. row0 = expert row offsets
// (exclusive prefix), grand = total rows. (One thread per expert would write
// a hot expert's hundreds of tiles alone.)
__device__ __forceinline__ void moe_write_tiles(const int32_t* tile0, const int32_t* row0, int grand, int E,
                                                int ntiles, int tile_t, int32_t* __restrict__ tiles) {
  for (int ti = threadIdx.x; ti < ntiles; ti += blockDim.x) {
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tile0[mid] <= ti) lo = mid;
      else hi = mid - 1;
    }
    const int total = (lo + 1 < E ? row0[lo + 1] : grand) - row0[lo];
    const int r = (ti - tile0[lo]) * tile_t;
    reinterpret_cast<int4*>(tiles)[ti] = int4{lo, row0[lo] + r, min(tile_t, total - r), 0};
  }
}

// counts[blk][e] = tokens of block blk routed to expert e.
__global__ __launch_bounds__(RBLK) void k_moe_count(const int32_t* __restrict__ idx, int32_t* __restrict__ counts,
                                                    int T, int K, int E) {
  __shared__ uint32_t bits[256 * BWS];
  const int blk = blockIdx.x;
  const int t0 = blk * RBLK;
  moe_block_bitmap(idx, bits, t0, min(RBLK, T - t0), K, E);
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < RBLK / 32; ++w) c += __popc(bits[e * BWS + w]);
    counts[(size_t)blk * E + e] = c;
  }
}

// One workgroup of 1024 threads: G = 1024 / E2 threads per expert (E2 = E
// rounded up to a power of two), thread (j, e) owning a contiguous range of
// blocks. Produces expert offsets, per-(block, expert) slot offsets and the
// grouped-GEMM tile list (expert, row0, rows).
constexpr int SCAN_THREADS = 1024;
__global__ __launch_bounds__(SCAN_THREADS) void k_moe_scan(const int32_t* __restrict__ counts,
                                                           int32_t* __restrict__ blk_off,
                                                           int32_t* __restrict__ expert_off,
                                                           int32_t* __restrict__ tiles,
                                                           int32_t* __restrict__ num_tiles, int nblk, int E, int E2,
                                                           int tile_t) {
  __shared__ int32_t part[SCAN_THREADS];  // [j][e] partial sums, then exclusive prefixes over j
  __shared__ int32_t tot[257], ntl[257];
  if (threadIdx.x < 256) {
    tot[threadIdx.x] = 0;
    ntl[threadIdx.x] = 0;
  }
  const int G = SCAN_THREADS / E2;
  const int e = threadIdx.x % E2, j = threadIdx.x / E2;
  const int per = (nblk + G - 1) / G;
  const int b0 = min(nblk, j * per), b1 = min(nblk, b0 + per);
  int sum = 0;
  // up to 8 blocks per thread (every shape up to 8 * G counting blocks): the
  // counts are loaded once, all in flight together, and kept for the offsets
  constexpr int PR = 8;
  const bool held = per <= PR;
  int cv[PR];
  if (held) {
#pragma unroll
    for (int u = 0; u < PR; ++u) cv[u] = (e < E && b0 + u < b1) ? counts[(size_t)(b0 + u) * E + e] : 0;
#pragma unroll
    for (int u = 0; u < PR; ++u) sum += cv[u];
  } else if (e < E) {
    int b = b0;
    for (; b + 8 <= b1; b += 8) {  // independent loads in flight
      int c[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) c[u] = counts[(size_t)(b + u) * E + e];
#pragma unroll
      for (int u = 0; u < 8; ++u) sum += c[u];
    }
    for (; b < b1; ++b) sum += counts[(size_t)b * E + e];
  }
  part[j * E2 + e] = sum;
  __syncthreads();
  if (j == 0) {  // exclusive prefix over j, per expert; totals
    int acc = 0;
    for (int jj = 0; jj < G; ++jj) {
      const int v = part[jj * E2 + e];
      part[jj * E2 + e] = acc;
      acc += v;
    }
    if (e < E) {
      tot[e] = acc;
      ntl[e] = (acc + tile_t - 1) / tile_t;
    }
  }
  __syncthreads();
  // exclusive scans over experts (E <= 256) by the first wave, 4 experts per lane
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    int c[4], n[4], cs = 0, ns = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      c[u] = tot[4 * l + u];
      n[u] = ntl[4 * l + u];
      cs += c[u];
      ns += n[u];
    }
    int ci = cs, ni = ns;  // inclusive scan of lane sums
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int a = __shfl_up(ci, o, 64), bb = __shfl_up(ni, o, 64);
      if (l >= o) {
        ci += a;
        ni += bb;
      }
    }
    int ce = ci - cs, ne = ni - ns;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      tot[4 * l + u] = ce;
      ntl[4 * l + u] = ne;
      ce += c[u];
      ne += n[u];
    }
    if (l == 63) {
      tot[256] = ce;  // grand total
      ntl[256] = ne;
      expert_off[E] = ce;
      *num_tiles = ne;
    }
  }
  __syncthreads();
  moe_write_tiles(ntl, tot, tot[256], E, ntl[256], tile_t, tiles);
  if (e < E) {
    const int base = tot[e];
    if (j == 0) expert_off[e] = base;
    int run = base + part[j * E2 + e];
    int b = held ? b1 : b0;
    if (held) {
#pragma unroll
      for (int u = 0; u < PR; ++u)
        if (b0 + u < b1) {
          blk_off[(size_t)(b0 + u) * E + e] = run;
          run += cv[u];
        }
    }
    for (; b + 8 <= b1; b += 8) {
      int c[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) c[u] = counts[(size_t)(b + u) * E + e];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        blk_off[(size_t)(b + u) * E + e] = run;
        run += c[u];
      }
    }
    for (; b < b1; ++b) {
      blk_off[(size_t)b * E + e] = run;
      run += counts[(size_t)b * E + e];
    }
  }
}

// Slot assignment: slot = blk_off[blk][e] + number of earlier tokens of the
// block routed to e (a popcount over the block bitmap). Within an expert the
// slots follow the token order (a token's K experts are distinct).
__global__ __launch_bounds__(RBLK) void k_moe_scatter(const int32_t* __restrict__ idx,
                                                      const int32_t* __restrict__ blk_off,
                                                      int32_t* __restrict__ slot_token, int32_t* __restrict__ slot_of,
                                                      int T, int K, int E) {
  __shared__ uint32_t bits[256 * BWS];
  const int blk = blockIdx.x;
  const int t0 = blk * RBLK;
  const int nt = min(RBLK, T - t0);
  moe_block_bitmap(idx, bits, t0, nt, K, E);
  __shared__ uint16_t pre[256 * BWS];
  moe_word_prefix(bits, pre, E);
  const int tl = threadIdx.x;
  if (tl >= nt) return;
  const int wl = tl >> 5;
  const uint32_t below = (1u << (tl & 31)) - 1u;
  for (int k = 0; k < K; ++k) {
    const size_t i = (size_t)(t0 + tl) * K + k;
    const int e = idx[i];
    if ((unsigned)e >= (unsigned)E) continue;
    const int rank = pre[e * BWS + wl] + __popc(bits[e * BWS + wl] & below);
    const int pos = blk_off[(size_t)blk * E + e] + rank;
    slot_token[pos] = t0 + tl;
    slot_of[i] = pos;
  }
}

// All three steps in one workgroup when every token fits one counting block
// (T <= RBLK): the bitmap, per-expert counts, the exclusive scans over
// experts (rows and tiles) and the slot assignment. Same outputs as the
// three kernels (expert_off, slot_token, slot_of, tiles, num_tiles; counts
// and blk_off are not written: nothing else reads them).
__global__ __launch_bounds__(RBLK) void k_moe_route_small(const int32_t* __restrict__ idx,
                                                          int32_t* __restrict__ expert_off,
                                                          int32_t* __restrict__ slot_token,
                                                          int32_t* __restrict__ slot_of, int32_t* __restrict__ tiles,
                                                          int32_t* __restrict__ num_tiles, int T, int K, int E,
                                                          int tile_t) {
  __shared__ uint32_t bits[256 * BWS];
  __shared__ int32_t off[256], toff[256], wsum[2][RBLK / 64];
  int ids[MAXK];  // this thread's token's expert ids, read once
  moe_load_ids(idx, 0, T, K, ids);
  moe_block_bitmap_ids(ids, bits, E);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // rows c and tiles n of expert e = tid; inclusive scans within the wave
  int c = 0;
  if (tid < E) {
#pragma unroll
    for (int w = 0; w < RBLK / 32; ++w) c += __popc(bits[tid * BWS + w]);
  }
  const int n = (c + tile_t - 1) / tile_t;
  int ci = c, ni = n;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int a = __shfl_up(ci, o, 64), bb = __shfl_up(ni, o, 64);
    if (lane >= o) {
      ci += a;
      ni += bb;
    }
  }
  if (lane == 63) {
    wsum[0][wv] = ci;
    wsum[1][wv] = ni;
  }
  __syncthreads();
  int cb = 0, nbase = 0, ct = 0, nt = 0;
#pragma unroll
  for (int w = 0; w < RBLK / 64; ++w) {
    cb += w < wv ? wsum[0][w] : 0;
    nbase += w < wv ? wsum[1][w] : 0;
    ct += wsum[0][w];
    nt += wsum[1][w];
  }
  const int base = cb + ci - c;  // exclusive prefix of rows
  if (tid < E) {
    off[tid] = base;
    toff[tid] = nbase + ni - n;  // exclusive prefix of tiles
    expert_off[tid] = base;
  }
  if (tid == 0) {
    expert_off[E] = ct;
    *num_tiles = nt;
  }
  __syncthreads();
  moe_write_tiles(toff, off, ct, E, nt, tile_t, tiles);
  __shared__ uint16_t pre[256 * BWS];
  moe_word_prefix(bits, pre, E);
  if (tid >= T) return;
  const int wl = tid >> 5;
  const uint32_t below = (1u << (tid & 31)) - 1u;
#pragma unroll
  for (int k = 0; k < MAXK; ++k) {
    const int e = ids[k];
    if ((unsigned)e >= (unsigned)E) continue;
    const size_t i = (size_t)tid * K + k;
    const int rank = pre[e * BWS + wl] + __popc(bits[e * BWS + wl] & below);
    const int pos = off[e] + rank;
    slot_token[pos] = tid;
    slot_of[i] = pos;
  }
}

// The same plan from per-tile expert counts, in one kernel instead of count,
// scan and scatter: counts[tile][e] holds the tokens of tile `tile` (tiles of
// RBLK / ct_per_blk rows) routed to expert e (the router GEMM's top-k
// epilogue writes them). Block blk sums, per expert, the counts of every tile
// (the expert's total) and of the tiles before its first token (its base
// within the expert), scans the totals over experts, and assigns its tokens'
// slots by bitmap ranks as k_moe_scatter does. Block 0 also writes
// expert_off, the tile list and num_tiles. Same outputs as the three kernels.
__global__ __launch_bounds__(RBLK) void k_moe_route_counts(const int32_t* __restrict__ idx,
                                                           const int32_t* __restrict__ counts, int n_ct,
                                                           int ct_per_blk, int32_t* __restrict__ expert_off,
                                                           int32_t* __restrict__ slot_token,
                                                           int32_t* __restrict__ slot_of, int32_t* __restrict__ tiles,
                                                           int32_t* __restrict__ num_tiles, int T, int K, int E,
                                                           int tile_t) {
  __shared__ uint32_t bits[256 * BWS];
  __shared__ int32_t psum[2][4 * RBLK];  // per (part of the tiles, expert): all tiles, tiles before the block
  __shared__ int32_t off[256], ebase[256], toff[256], wsum[2][RBLK / 64];
  __shared__ uint16_t pre[256 * BWS];
  const int blk = blockIdx.x, t0 = blk * RBLK, ntok = min(RBLK, T - t0);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // this thread's token's expert ids, issued before the count loads so both
  // latencies overlap, and kept for the slot assignment
  int ids[MAXK];
  moe_load_ids(idx, t0, ntok, K, ids);
  // Per-expert sums over the tiles, in G parts of the tile range. With E a
  // multiple of 4 a thread loads 16 bytes (4 experts' counts) per tile:
  // E2 / 4 expert groups x G = 4 RBLK / E2 parts; otherwise one expert per
  // thread: E2 experts x G = RBLK / E2 parts (E2: E rounded up to 64, 128 or
  // 256). Loads are issued 16 at a time with addresses clamped into the
  // array and values past the range dropped.
  const int E2 = E <= 64 ? 64 : (E <= 128 ? 128 : 256);
  const bool vec = (E & 3) == 0;
  const int G = vec ? 4 * RBLK / E2 : RBLK / E2;
  {
    const int tb = blk * ct_per_blk;
    const int lanes = vec ? E2 / 4 : E2;  // threads per part
    const int e0 = vec ? 4 * (tid % lanes) : tid % lanes, q = tid / lanes;
    const int per = (n_ct + G - 1) / G, lo = min(n_ct, q * per), hi = min(n_ct, lo + per);
    int sa[4] = {0, 0, 0, 0}, sb[4] = {0, 0, 0, 0};
    if (vec) {
      const int ec = min(e0, E - 4);
      for (int t = lo; t < hi; t += 16) {
        int4 c[16];
#pragma unroll
        for (int u = 0; u < 16; ++u)
          c[u] = *reinterpret_cast<const int4*>(counts + (size_t)min(t + u, n_ct - 1) * E + ec);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const bool in = t + u < hi && e0 < E, before = t + u < tb;
          const int v[4] = {c[u].x, c[u].y, c[u].z, c[u].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            sa[i] += in ? v[i] : 0;
            sb[i] += in && before ? v[i] : 0;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        psum[0][q * E2 + e0 + i] = sa[i];
        psum[1][q * E2 + e0 + i] = sb[i];
      }
    } else {
      const int ec = min(e0, E - 1);
      for (int t = lo; t < hi; t += 16) {
        int c[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) c[u] = counts[(size_t)min(t + u, n_ct - 1) * E + ec];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int v = t + u < hi && e0 < E ? c[u] : 0;
          sa[0] += v;
          sb[0] += t + u < tb ? v : 0;
        }
      }
      psum[0][q * E2 + e0] = sa[0];
      psum[1][q * E2 + e0] = sb[0];
    }
  }
  moe_block_bitmap_ids(ids, bits, E);  // (its barriers also publish psum)
  // rows c and tiles n of expert e = tid; inclusive scans within the wave
  int c = 0, below = 0;
  if (tid < E) {
    for (int q = 0; q < G; ++q) {
      c += psum[0][q * E2 + tid];
      below += psum[1][q * E2 + tid];
    }
  }
  const int n = (c + tile_t - 1) / tile_t;
  int ci = c, ni = n;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int a = __shfl_up(ci, o, 64), bb = __shfl_up(ni, o, 64);
    if (lane >= o) {
      ci += a;
      ni += bb;
    }
  }
  if (lane == 63) {
    wsum[0][wv] = ci;
    wsum[1][wv] = ni;
  }
  __syncthreads();
  int cb = 0, nbase = 0, ct = 0, nt = 0;
#pragma unroll
  for (int w = 0; w < RBLK / 64; ++w) {
    cb += w < wv ? wsum[0][w] : 0;
    nbase += w < wv ? wsum[1][w] : 0;
    ct += wsum[0][w];
    nt += wsum[1][w];
  }
  const int base = cb + ci - c;  // exclusive prefix of rows
  if (tid < E) {
    ebase[tid] = base;
    off[tid] = base + below;
    toff[tid] = nbase + ni - n;  // exclusive prefix of tiles
    if (blk == 0) expert_off[tid] = base;
  }
  if (blk == 0 && tid == 0) {
    expert_off[E] = ct;
    *num_tiles = nt;
  }
  __syncthreads();
  if (blk == 0) moe_write_tiles(toff, ebase, ct, E, nt, tile_t, tiles);
  moe_word_prefix(bits, pre, E);
  if (tid >= ntok) return;
  const int wl = tid >> 5;
  const uint32_t lower = (1u << (tid & 31)) - 1u;
#pragma unroll
  for (int k = 0; k < MAXK; ++k) {
    const int e = ids[k];
    if ((unsigned)e >= (unsigned)E) continue;
    const size_t i = (size_t)(t0 + tid) * K + k;
    const int rank = pre[e * BWS + wl] + __popc(bits[e * BWS + wl] & lower);
    const int pos = off[e] + rank;
    slot_token[pos] = t0 + tid;
    slot_of[i] = pos;
  }
}

// ----------------------------------------------------------------------------
// MoE combine (scatter_add_weighted_f32 :1027-1055 + cast_f32_to_fp16_scaled
// :1153-1164 + add_fp16). Each token sums its K expert outputs in ascending
// expert id — the order the reference's expert-major loop adds them — with
// fused multiply-adds, then rounds to fp16 and adds the residual.
// The reference weights by softmax/K and rescales by K at the end; both are
// exact powers of two, so weighting by the softmax directly is bit-identical.
// NMODE: -1 = no norm; OUT_F16 / OUT_SPLIT = form of the next block's norm output.
// NJ 256-element slices per row (3 covers D <= 768 with fewer registers
// than the general 4, so more waves stay resident).
// Y16: the expert outputs are fp16 (the fp16 numerics' down GEMM rounds them
// once; widened here by the hardware), else f32.
template <int NMODE, int K, int NJ = MAXJ, bool Y16 = false, bool RES = true>
__global__ __launch_bounds__(256) void k_moe_combine(const int32_t* __restrict__ idx, const float* __restrict__ w,
                                                     const int32_t* __restrict__ slot_of, const void* __restrict__ y,
                                                     const uint16_t* __restrict__ residual,
                                                     uint16_t* __restrict__ moe_out, uint16_t* __restrict__ h_out,
                                                     const uint16_t* __restrict__ gamma,
                                                     uint16_t* __restrict__ norm_hi, uint16_t* __restrict__ norm_lo,
                                                     int T, int D, float eps) {
  const int t = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (t >= T) return;
  moe_combine_row<NMODE, K, NJ, Y16, RES>(t, threadIdx.x & 63, idx, w, slot_of, y, residual, moe_out, h_out, gamma,
                                          norm_hi, norm_lo, D, eps);
}

template <int NMODE, bool Y16, bool RES>
void launch_combine_t(pfhip_backend* b, const int32_t* idx, const float* w, const int32_t* slot_of, const void* y,
                      const uint16_t* residual, uint16_t* moe_out, uint16_t* h_out, const uint16_t* gamma,
                      uint16_t* norm_hi, uint16_t* norm_lo, int T, int K, int D, float eps) {
  const dim3 grid((T + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK);
  if (Y16 || (D <= 768 && K == 4)) {  // the model's shape (fp16 expert outputs are built for it only)
    PF_CHECK(K == 4 && D <= 768, "moe_combine: fp16 expert outputs are built for K = 4, D <= 768");
    hipLaunchKernelGGL((k_moe_combine<NMODE, 4, 3, Y16, RES>), grid, dim3(256), 0, b->stream, idx, w, slot_of, y,
                       residual, moe_out, h_out, gamma, norm_hi, norm_lo, T, D, eps);
    PF_HIP(hipGetLastError());
    return;
  }
  switch (K) {
#define PF_COMBINE_CASE(k)                                                                                         \
  case k:                                                                                                          \
    hipLaunchKernelGGL((k_moe_combine<NMODE, k, MAXJ, false, RES>), grid, dim3(256), 0, b->stream, idx, w, slot_of, \
                       y, residual, moe_out, h_out, gamma, norm_hi, norm_lo, T, D, eps);                           \
    break;
    PF_COMBINE_CASE(1) PF_COMBINE_CASE(2) PF_COMBINE_CASE(3) PF_COMBINE_CASE(4)
    PF_COMBINE_CASE(5) PF_COMBINE_CASE(6) PF_COMBINE_CASE(7) PF_COMBINE_CASE(8)
#undef PF_COMBINE_CASE
    default: throw Error("moe_combine: K must be 1..8");
  }
  PF_HIP(hipGetLastError());
}

// residual NULL: no residual (a variant that loads none)
template <int NMODE>
void launch_combine(pfhip_backend* b, const int32_t* idx, const float* w, const int32_t* slot_of, const void* y,
                    bool y16, const uint16_t* residual, uint16_t* moe_out, uint16_t* h_out, const uint16_t* gamma,
                    uint16_t* norm_hi, uint16_t* norm_lo, int T, int K, int D, float eps) {
  if (y16) {
    if (residual)
      launch_combine_t<NMODE, true, true>(b, idx, w, slot_of, y, residual, moe_out, h_out, gamma, norm_hi, norm_lo, T,
                                          K, D, eps);
    else
      launch_combine_t<NMODE, true, false>(b, idx, w, slot_of, y, residual, moe_out, h_out, gamma, norm_hi, norm_lo,
                                           T, K, D, eps);
  } else {
    if (residual)
      launch_combine_t<NMODE, false, true>(b, idx, w, slot_of, y, residual, moe_out, h_out, gamma, norm_hi, norm_lo,
                                           T, K, D, eps);
    else
      launch_combine_t<NMODE, false, false>(b, idx, w, slot_of, y, residual, moe_out, h_out, gamma, norm_hi, norm_lo,
                                            T, K, D, eps);
  }
}

// ----------------------------------------------------------------------------
// fp16-weight router (router W fp16 [D][E], f32
// accumulate, fp16 bias): logits[t][e] = sum_d x[t][d] W[d][e] + bias[e], on
// the matrix cores. W is first transposed into wt [E][D] (a scratch copy) so
// that every MFMA operand is one 16-byte load: A = W^T (16 experts x 32 k),
// B = x^T (32 k x 16 tokens); a lane ends with 4 consecutive experts of one
// token. One wave per 16 tokens and 32 experts (many small workgroups: the
// GEMM is tiny and its K loop is a chain of L2 loads); operands come straight
// from global memory (W^T is 160 KB and L2-resident).
__global__ __launch_bounds__(256) void k_transpose_f16(const uint16_t* __restrict__ w, uint16_t* __restrict__ wt,
                                                       int D, int E) {
  __shared__ uint16_t tile[32][33];
  const int e0 = blockIdx.x * 32, d0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int r = ty; r < 32; r += 8) {
    const int d = d0 + r, e = e0 + tx;
    tile[r][tx] = (d < D && e < E) ? w[(size_t)d * E + e] : (uint16_t)0;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int e = e0 + r, d = d0 + tx;
    if (e < E && d < D) wt[(size_t)e * D + d] = tile[tx][r];
  }
}

__global__ __launch_bounds__(64) void k_router_f16w(const uint16_t* __restrict__ x, const uint16_t* __restrict__ wt,
                                                    const uint16_t* __restrict__ bias, float* __restrict__ logits,
                                                    int T, int D, int E) {
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int t0 = blockIdx.x * 16, eb = blockIdx.y * 32;
  const uint16_t* arow[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) arow[f] = wt + (size_t)min(eb + 16 * f + l16, E - 1) * D + 8 * lg;
  const uint16_t* brow = x + (size_t)min(t0 + l16, T - 1) * D + 8 * lg;
  f4_t acc[2] = {f4_t{0.f, 0.f, 0.f, 0.f}, f4_t{0.f, 0.f, 0.f, 0.f}};
  for (int k = 0; k < D; k += 32) {
    const h8_t a0 = __builtin_bit_cast(h8_t, *reinterpret_cast<const u4_t*>(arow[0] + k));
    const h8_t a1 = __builtin_bit_cast(h8_t, *reinterpret_cast<const u4_t*>(arow[1] + k));
    const h8_t bb = __builtin_bit_cast(h8_t, *reinterpret_cast<const u4_t*>(brow + k));
    acc[0] = mfma16x16x32(a0, bb, acc[0]);
    acc[1] = mfma16x16x32(a1, bb, acc[1]);
  }
  const int t = t0 + l16;
  if (t >= T) return;
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const int e = eb + 16 * f + 4 * lg;
    float* o = logits + (size_t)t * E + e;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (e + r < E) o[r] = acc[f][r] + (bias ? hw_h2f(bias[e + r]) : 0.0f);
  }
}

// ----------------------------------------------------------------------------
// Reference-layout QMoE kernels (native/shaders/qmoe_gate_up.wgsl,
// qmoe_down_scatter.wgsl) for the named-dispatch surface: one thread per
// (t*K + k, n). The down variant accumulates a token's K contributions in k
// order into `acc` (deterministic; the WGSL uses CAS atomics).
__device__ float dot_int4_row(const float* x, const uint8_t* wrow, const uint16_t* srow, const uint8_t* zrow, int D) {
  const int nb = D >> 5;
  float acc = 0.0f;
  for (int b = 0; b < nb; ++b) {
    const float sc = wasm_h2f(srow[b]);
    int z = 0;
    if (zrow) { const uint8_t zb = zrow[b >> 1]; z = (b & 1) ? (zb >> 4) : (zb & 0xF); }
    float bs = 0.0f;
    for (int j = 0; j < 16; ++j) {
      const uint8_t by = wrow[b * 16 + j];
      bs = fmaf((float)((int)(by & 0xF) - z), x[b * 32 + 2 * j], bs);
      bs = fmaf((float)((int)(by >> 4) - z), x[b * 32 + 2 * j + 1], bs);
    }
    acc = fmaf(bs, sc, acc);
  }
  return acc;
}

__global__ void k_qmoe_gate_up(const float* x, const int32_t* ridx, const uint8_t* w, const uint16_t* ws,
                               const uint8_t* wz, const uint16_t* bias, float* out, int T, int K, int N, int D) {
  const int tk = blockIdx.x;
  const int n = blockIdx.y * blockDim.x + threadIdx.x;
  if (tk >= T * K || n >= N) return;
  const int t = tk / K, e = ridx[tk];
  const int nb = D >> 5, zs = (nb + 1) >> 1;
  const size_t r = (size_t)e * N + n;
  const float v = dot_int4_row(x + (size_t)t * D, w + r * (D >> 1), ws + r * nb, wz ? wz + r * zs : nullptr, D);
  out[(size_t)tk * N + n] = v + (bias ? wasm_h2f(bias[r]) : 0.0f);
}

__global__ void k_qmoe_down(const float* glu, const int32_t* ridx, const float* rw, const uint8_t* w,
                            const uint16_t* ws, const uint8_t* wz, const uint16_t* bias, float* acc, int T, int K,
                            int N, int D) {
  const int t = blockIdx.x;
  const int n = blockIdx.y * blockDim.x + threadIdx.x;
  if (t >= T || n >= N) return;
  const int nb = D >> 5, zs = (nb + 1) >> 1;
  float a = acc[(size_t)t * N + n];
  for (int k = 0; k < K; ++k) {
    const int tk = t * K + k, e = ridx[tk];
    const size_t r = (size_t)e * N + n;
    float v = dot_int4_row(glu + (size_t)tk * D, w + r * (D >> 1), ws + r * nb, wz ? wz + r * zs : nullptr, D);
    v = v + (bias ? wasm_h2f(bias[r]) : 0.0f);
    a = a + rw[tk] * v;
  }
  acc[(size_t)t * N + n] = a;
}

unsigned grid1d(size_t n, int block = 256) {
  size_t g = (n + block - 1) / block;
  if (g > 65535u * 16u) g = 65535u * 16u;
  return (unsigned)(g ? g : 1);
}

// ----------------------------------------------------------------------------
// Test probes. Each walks the f32 bit patterns [lo, hi) and counts the inputs
// where a fast routine and the formulation it replaces disagree bit-wise:
// out[0] = mismatches, out[1] = smallest mismatching pattern (init 0xFFFFFFFF),
// out[2] = inputs outside the routine's stated domain that differ.
__global__ void k_probe_div_one_plus(uint32_t lo, uint32_t hi, uint32_t* out) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint32_t bad = 0, first = 0xFFFFFFFFu;
  for (uint64_t i = lo + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < hi; i += stride) {
    const float e = __uint_as_float((uint32_t)i);
    const float fast = div_one_plus(e);
    const float ieee = e / (1.0f + e);
    if (__float_as_uint(fast) != __float_as_uint(ieee)) {
      ++bad;
      first = min(first, (uint32_t)i);
    }
  }
  if (bad) {
    atomicAdd(&out[0], bad);
    atomicMin(&out[1], first);
  }
}

// x = -(pattern as f32) for patterns of non-negative finite floats: every
// x <= 0. Inputs with floor(max(x, -88) log2 e) = -127 are counted in out[2].
__global__ void k_probe_exp_fast(uint32_t lo, uint32_t hi, uint32_t* out) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint32_t bad = 0, first = 0xFFFFFFFFu, outside = 0;
  for (uint64_t i = lo + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < hi; i += stride) {
    const float x = -__uint_as_float((uint32_t)i);
    const float y = fmaxf(x, -88.0f) * 1.44269504088896340736f;
    const bool edge = floorf(y) < -126.0f;
    if (__float_as_uint(exp_approx_fast(x)) != __float_as_uint(exp_approx(x))) {
      if (edge) {
        ++outside;
      } else {
        ++bad;
        first = min(first, (uint32_t)i);
      }
    }
  }
  if (bad) {
    atomicAdd(&out[0], bad);
    atomicMin(&out[1], first);
  }
  if (outside) atomicAdd(&out[2], outside);
}

// Plain 16-byte copy (the known-size workload the HBM counters are scaled by).
__global__ void k_copy16(const u4_t* __restrict__ src, u4_t* __restrict__ dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

// The same copy with the loads going HBM -> LDS directly
// (global_load_lds_dwordx4, as the GEMMs load their activations), then LDS ->
// registers -> HBM: the counters' factor for that load form.
__global__ __launch_bounds__(256) void k_copy16_lds(const u4_t* __restrict__ src, u4_t* __restrict__ dst, size_t n) {
  __shared__ __attribute__((aligned(16))) u4_t stage[256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (size_t base = (size_t)blockIdx.x * 256; base < n; base += (size_t)gridDim.x * 256) {
    const size_t i = min(base + threadIdx.x, n - 1);  // lanes past n re-read the last unit (not stored)
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(src + i, (__attribute__((address_space(3))) void*)(stage + wave * 64), 16, 0, 0);
#endif
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (base + threadIdx.x < n) dst[base + threadIdx.x] = stage[wave * 64 + lane];
    __syncthreads();
  }
}

// dst[i] = table[idx[i]] in 16-byte units: scattered 16-byte reads, as the
// embedding gather and the expert GEMMs' row gathers make them.
__global__ void k_gather16(const u4_t* __restrict__ table, const int32_t* __restrict__ idx, u4_t* __restrict__ dst,
                           size_t n, uint32_t table_units) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = table[(uint32_t)idx[i] % table_units];
}

}  // namespace

void copy16_lds(pfhip_backend* b, const void* src, void* dst, size_t bytes) {
  PF_CHECK(bytes % 16 == 0 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0,
           "copy16_lds: 16-byte aligned sizes and pointers");
  if (!bytes) return;
  ProfScope ps(b, "copy16_lds");
  hipLaunchKernelGGL(k_copy16_lds, dim3(4096), dim3(256), 0, b->stream, static_cast<const u4_t*>(src),
                     static_cast<u4_t*>(dst), bytes / 16);
  PF_HIP(hipGetLastError());
}

void gather16(pfhip_backend* b, const void* table, uint32_t table_units, const int32_t* idx, void* dst, size_t n) {
  PF_CHECK(table_units > 0 && ((uintptr_t)table & 15) == 0 && ((uintptr_t)dst & 15) == 0,
           "gather16: 16-byte aligned table and output, non-empty table");
  if (!n) return;
  ProfScope ps(b, "gather16");
  hipLaunchKernelGGL(k_gather16, dim3(4096), dim3(256), 0, b->stream, static_cast<const u4_t*>(table), idx,
                     static_cast<u4_t*>(dst), n, table_units);
  PF_HIP(hipGetLastError());
}

void copy16(pfhip_backend* b, const void* src, void* dst, size_t bytes) {
  PF_CHECK(bytes % 16 == 0 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0,
           "copy16: 16-byte aligned sizes and pointers");
  if (!bytes) return;
  ProfScope ps(b, "copy16");
  hipLaunchKernelGGL(k_copy16, dim3(4096), dim3(256), 0, b->stream, static_cast<const u4_t*>(src),
                     static_cast<u4_t*>(dst), bytes / 16);
  PF_HIP(hipGetLastError());
}

// Hardware exp2 (v_exp_f32) on x = -(pattern as f32) against exp2 evaluated
// in double and rounded to f32: out[0] = largest difference in f32 ulps,
// out[1] = inputs more than 1 ulp off, out[2] = inputs more than 4 ulps off.
// Inputs whose exact result is below the smallest normal f32 are skipped.
__global__ void k_probe_exp2_hw(uint32_t lo, uint32_t hi, uint32_t* out) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint32_t worst = 0, over1 = 0, over4 = 0;
  for (uint64_t i = lo + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < hi; i += stride) {
    const float x = -__uint_as_float((uint32_t)i);
    if (!(x >= -126.0f)) continue;
    const float hw = __builtin_amdgcn_exp2f(x);
    const float ref = (float)exp2((double)x);
    const int32_t d = (int32_t)__float_as_uint(hw) - (int32_t)__float_as_uint(ref);
    const uint32_t ad = (uint32_t)(d < 0 ? -d : d);
    worst = max(worst, ad);
    over1 += ad > 1;
    over4 += ad > 4;
  }
  atomicMax(&out[0], worst);
  if (over1) atomicAdd(&out[1], over1);
  if (over4) atomicAdd(&out[2], over4);
}

void probe_fast_math(pfhip_backend* b, int which, uint32_t lo, uint32_t hi, uint32_t* out) {
  PF_CHECK(lo <= hi, "probe_fast_math: empty range");
  ProfScope ps(b, "probe_fast_math");
  if (which == 0)
    hipLaunchKernelGGL(k_probe_div_one_plus, dim3(8192), dim3(256), 0, b->stream, lo, hi, out);
  else if (which == 1)
    hipLaunchKernelGGL(k_probe_exp_fast, dim3(8192), dim3(256), 0, b->stream, lo, hi, out);
  else
    hipLaunchKernelGGL(k_probe_exp2_hw, dim3(8192), dim3(256), 0, b->stream, lo, hi, out);
  PF_HIP(hipGetLastError());
}

void embed_lookup(pfhip_backend* b, const uint8_t* q, const uint16_t* s, const uint8_t* zp, const int32_t* ids,
                  uint16_t* out, int T, int V, int D, bool stream_out) {
  PF_CHECK(D > 0 && D % 32 == 0, "embed_lookup: D must be a multiple of 32");
  PF_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)out & 15) == 0,
           "embed_lookup: table and output must be 16-byte aligned");
  if (T <= 0) return;
  const size_t n = (size_t)((T + EMB_TOK - 1) / EMB_TOK) * (D / 8);
  PF_CHECK(n < (1ull << 31), "embed_lookup: too many rows");
  ProfScope ps(b, "embed_lookup_int4");
  if (stream_out)
    hipLaunchKernelGGL(k_embed<true>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, b->stream, q, s, zp, ids, out,
                       T, V, D);
  else
    hipLaunchKernelGGL(k_embed<false>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, b->stream, q, s, zp, ids, out,
                       T, V, D);
  PF_HIP(hipGetLastError());
}

void embed_rms_norm_f16(pfhip_backend* b, const uint8_t* q, const uint16_t* s, const uint8_t* zp, const int32_t* ids,
                        const uint16_t* g, uint16_t* h, uint16_t* out, int T, int V, int D, float eps) {
  const bool fused = D == 640 && ((reinterpret_cast<uintptr_t>(q) & 3) | ((reinterpret_cast<uintptr_t>(g) |
                                   reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(out)) & 15)) == 0;
  if (!fused) {
    embed_lookup(b, q, s, zp, ids, h, T, V, D);
    rms_norm_f16(b, h, g, out, T, D, eps);
    return;
  }
  if (T <= 0) return;
  ProfScope ps(b, "embed_rms_norm");
  hipLaunchKernelGGL(k_embed_rms_norm4<5>, dim3((unsigned)((T + 15) / 16)), dim3(256), 0, b->stream, q, s, zp, ids, g,
                     h, out, T, V, eps);
  PF_HIP(hipGetLastError());
}

void rms_norm_f16(pfhip_backend* b, const uint16_t* x, const uint16_t* g, uint16_t* out, int T, int D, float eps) {
  PF_CHECK(D > 0 && D % 4 == 0 && D <= 256 * MAXJ, "rms_norm: D must be a multiple of 4, at most 1024");
  if (T <= 0) return;
  ProfScope ps(b, "rms_norm");
  const bool al16 = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(g) |
                      reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  const dim3 g16((T + 15) / 16);  // 4 waves x 4 rows per block
  if (al16 && D == 640) hipLaunchKernelGGL(k_rms_norm4<5>, g16, dim3(256), 0, b->stream, x, g, out, T, eps);
  else if (al16 && D == 512) hipLaunchKernelGGL(k_rms_norm4<4>, g16, dim3(256), 0, b->stream, x, g, out, T, eps);
  else if (al16 && D == 768) hipLaunchKernelGGL(k_rms_norm4<6>, g16, dim3(256), 0, b->stream, x, g, out, T, eps);
  else hipLaunchKernelGGL(k_rms_norm<OUT_F16>, dim3((T + 3) / 4), dim3(256), 0, b->stream, x, g, out, nullptr, T, D, eps);
  PF_HIP(hipGetLastError());
}

void rms_norm_f32(pfhip_backend* b, const uint16_t* x, const uint16_t* g, float* out, int T, int D, float eps) {
  PF_CHECK(D > 0 && D % 4 == 0 && D <= 256 * MAXJ, "rms_norm: D must be a multiple of 4, at most 1024");
  if (T <= 0) return;
  ProfScope ps(b, "rms_norm_fp16_to_f32");
  hipLaunchKernelGGL(k_rms_norm<OUT_F32>, dim3((T + 3) / 4), dim3(256), 0, b->stream, x, g, out, nullptr, T, D, eps);
  PF_HIP(hipGetLastError());
}

void rms_norm_split(pfhip_backend* b, const uint16_t* x, const uint16_t* g, uint16_t* hi, uint16_t* lo, int T, int D,
                    float eps) {
  PF_CHECK(D > 0 && D % 4 == 0 && D <= 256 * MAXJ, "rms_norm: D must be a multiple of 4, at most 1024");
  if (T <= 0) return;
  ProfScope ps(b, "rms_norm_split");
  hipLaunchKernelGGL(k_rms_norm<OUT_SPLIT>, dim3((T + 3) / 4), dim3(256), 0, b->stream, x, g, hi, lo, T, D, eps);
  PF_HIP(hipGetLastError());
}

void add_rms_norm_f32(pfhip_backend* b, const uint16_t* a, const uint16_t* bb, const uint16_t* g, uint16_t* sum_out,
                      float* norm_out, int T, int D, float eps) {
  PF_CHECK(D > 0 && D % 4 == 0 && D <= 256 * MAXJ, "add_rmsnorm: D must be a multiple of 4, at most 1024");
  if (T <= 0) return;
  ProfScope ps(b, "add_rmsnorm_fp16_to_f32");
  hipLaunchKernelGGL(k_add_rms_norm<OUT_F32>, dim3((T + 3) / 4), dim3(256), 0, b->stream, a, bb, g, sum_out,
                     norm_out, nullptr, T, D, eps);
  PF_HIP(hipGetLastError());
}

void add_rms_norm_f16(pfhip_backend* b, const uint16_t* a, const uint16_t* bb, const uint16_t* g, uint16_t* sum_out,
                      uint16_t* norm_out, int T, int D, float eps) {
  PF_CHECK(D > 0 && D % 4 == 0 && D <= 256 * MAXJ, "add_rmsnorm: D must be a multiple of 4, at most 1024");
  if (T <= 0) return;
  ProfScope ps(b, "add_rmsnorm_f16");
  hipLaunchKernelGGL(k_add_rms_norm<OUT_F16>, dim3((T + 3) / 4), dim3(256), 0, b->stream, a, bb, g, sum_out,
                     norm_out, nullptr, T, D, eps);
  PF_HIP(hipGetLastError());
}

void add_rms_norm_split(pfhip_backend* b, const uint16_t* a, const uint16_t* bb, const uint16_t* g,
                        uint16_t* sum_out, uint16_t* hi, uint16_t* lo, int T, int D, float eps) {
  PF_CHECK(D > 0 && D % 4 == 0 && D <= 256 * MAXJ, "add_rmsnorm: D must be a multiple of 4, at most 1024");
  if (T <= 0) return;
  ProfScope ps(b, "add_rmsnorm_split");
  hipLaunchKernelGGL(k_add_rms_norm<OUT_SPLIT>, dim3((T + 3) / 4), dim3(256), 0, b->stream, a, bb, g, sum_out, hi,
                     lo, T, D, eps);
  PF_HIP(hipGetLastError());
}

void split_f32(pfhip_backend* b, const float* x, uint16_t* hi, uint16_t* lo, size_t n) {
  if (!n) return;
  ProfScope ps(b, "split_f32");
  hipLaunchKernelGGL(k_split_f32, dim3(grid1d(n)), dim3(256), 0, b->stream, x, hi, lo, n);
  PF_HIP(hipGetLastError());
}

void add_f16(pfhip_backend* b, const uint16_t* a, const uint16_t* bb, uint16_t* out, size_t n) {
  if (!n) return;
  ProfScope ps(b, "add_fp16");
  hipLaunchKernelGGL(k_add_f16, dim3(grid1d(n)), dim3(256), 0, b->stream, a, bb, out, n);
  PF_HIP(hipGetLastError());
}
void cast_f16_f32(pfhip_backend* b, const uint16_t* s, float* d, size_t n) {
  if (!n) return;
  ProfScope ps(b, "cast_fp16_to_f32");
  hipLaunchKernelGGL(k_cast_f16_f32, dim3(grid1d(n)), dim3(256), 0, b->stream, s, d, n);
  PF_HIP(hipGetLastError());
}
void cast_f16_f32_ieee(pfhip_backend* b, const uint16_t* s, float* d, size_t n) {
  if (!n) return;
  ProfScope ps(b, "cast_logits_f32");
  hipLaunchKernelGGL(k_cast_f16_f32_ieee, dim3(grid1d(n)), dim3(256), 0, b->stream, s, d, n);
  PF_HIP(hipGetLastError());
}
void cast_f32_f16_scaled(pfhip_backend* b, const float* s, uint16_t* d, size_t n, float scale) {
  if (!n) return;
  ProfScope ps(b, "cast_f32_to_fp16_scaled");
  hipLaunchKernelGGL(k_cast_f32_f16_scaled, dim3(grid1d(n)), dim3(256), 0, b->stream, s, d, n, scale);
  PF_HIP(hipGetLastError());
}
void zero_f32(pfhip_backend* b, float* p, size_t n) {
  if (!n) return;
  ProfScope ps(b, "zero_f32");
  hipLaunchKernelGGL(k_zero_f32, dim3(grid1d(n)), dim3(256), 0, b->stream, p, n);
  PF_HIP(hipGetLastError());
}
void swiglu_f32(pfhip_backend* b, const float* gu, float* out, int rows, int dff) {
  if (rows <= 0 || dff <= 0) return;
  ProfScope ps(b, "swiglu_clamp");
  hipLaunchKernelGGL(k_swiglu, dim3(grid1d((size_t)rows * dff)), dim3(256), 0, b->stream, gu, out, rows, dff);
  PF_HIP(hipGetLastError());
}
void rope_apply(pfhip_backend* b, uint16_t* qk, const uint16_t* c, const uint16_t* s, int T, int H, int hd,
                int row_stride, int seq_len) {
  PF_CHECK(hd % 2 == 0 && seq_len > 0, "rope_apply: bad shape");
  if (T <= 0) return;
  ProfScope ps(b, "rope_apply");
  hipLaunchKernelGGL(k_rope, dim3(grid1d((size_t)T * H * (hd / 2))), dim3(256), 0, b->stream, qk, c, s, T, H, hd,
                     row_stride, seq_len);
  PF_HIP(hipGetLastError());
}

void router_topk(pfhip_backend* b, const float* logits, int32_t* idx, float* w, int T, int E, int K, float wscale) {
  PF_CHECK(K >= 1 && K <= MAXK && K <= E, "router_topk: need 1 <= K <= min(8, E)");
  if (T <= 0) return;
  PF_CHECK(E <= 64 * TOPK_PL, "router_topk: E must be at most 256");
  ProfScope ps(b, "router_topk");
  const dim3 grid((T + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK);
  switch (K) {
#define PF_TOPK_CASE(k) \
  case k: hipLaunchKernelGGL(k_router_topk<k>, grid, dim3(256), 0, b->stream, logits, idx, w, T, E, wscale); break;
    PF_TOPK_CASE(1) PF_TOPK_CASE(2) PF_TOPK_CASE(3) PF_TOPK_CASE(4)
    PF_TOPK_CASE(5) PF_TOPK_CASE(6) PF_TOPK_CASE(7) PF_TOPK_CASE(8)
#undef PF_TOPK_CASE
  }
  PF_HIP(hipGetLastError());
}

int moe_max_tiles(int T, int K, int E, int tile_t) { return (T * K + tile_t - 1) / tile_t + E; }

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t moe_plan_bytes(int T, int K, int E, int tile_t) {
  const size_t nblk = (size_t)(T + RBLK - 1) / RBLK;
  return al256(nblk * E * 4) * 2 + al256((size_t)(E + 1) * 4) + al256((size_t)T * K * 4) * 2 +
         al256((size_t)moe_max_tiles(T, K, E, tile_t) * 16) + 256 + al256((size_t)(T + 15) / 16 * E * 4);
}

MoePlan moe_plan_carve(void* base, int T, int K, int E, int tile_t) {
  const size_t nblk = (size_t)(T + RBLK - 1) / RBLK;
  char* p = static_cast<char*>(base);
  MoePlan m;
  m.counts = reinterpret_cast<int32_t*>(p); p += al256(nblk * E * 4);
  m.blk_off = reinterpret_cast<int32_t*>(p); p += al256(nblk * E * 4);
  m.expert_off = reinterpret_cast<int32_t*>(p); p += al256((size_t)(E + 1) * 4);
  m.slot_token = reinterpret_cast<int32_t*>(p); p += al256((size_t)T * K * 4);
  m.slot_of = reinterpret_cast<int32_t*>(p); p += al256((size_t)T * K * 4);
  m.tiles = reinterpret_cast<int32_t*>(p); p += al256((size_t)moe_max_tiles(T, K, E, tile_t) * 16);
  m.num_tiles = reinterpret_cast<int32_t*>(p); p += 256;
  m.tile_counts = reinterpret_cast<int32_t*>(p);
  m.max_tiles = moe_max_tiles(T, K, E, tile_t);
  m.tile_t = tile_t;
  return m;
}

void moe_route(pfhip_backend* b, const int32_t* idx, int T, int K, int E, const MoePlan& m) {
  PF_CHECK(E >= 1 && E <= 256 && K >= 1 && K <= MAXK, "moe_route: need E <= 256 and K <= 8");
  if (T <= 0) return;
  const int nblk = (T + RBLK - 1) / RBLK;
  if (nblk == 1) {
    ProfScope ps(b, "moe_route");
    hipLaunchKernelGGL(k_moe_route_small, dim3(1), dim3(RBLK), 0, b->stream, idx, m.expert_off, m.slot_token,
                       m.slot_of, m.tiles, m.num_tiles, T, K, E, m.tile_t);
    PF_HIP(hipGetLastError());
    return;
  }
  {
    ProfScope ps(b, "moe_count");
    hipLaunchKernelGGL(k_moe_count, dim3(nblk), dim3(RBLK), 0, b->stream, idx, m.counts, T, K, E);
    PF_HIP(hipGetLastError());
  }
  {
    ProfScope ps(b, "moe_scan");
    int E2 = 1;
    while (E2 < E) E2 <<= 1;
    hipLaunchKernelGGL(k_moe_scan, dim3(1), dim3(SCAN_THREADS), 0, b->stream, m.counts, m.blk_off, m.expert_off,
                       m.tiles, m.num_tiles, nblk, E, E2, m.tile_t);
    PF_HIP(hipGetLastError());
  }
  {
    ProfScope ps(b, "moe_scatter");
    hipLaunchKernelGGL(k_moe_scatter, dim3(nblk), dim3(RBLK), 0, b->stream, idx, m.blk_off, m.slot_token, m.slot_of,
                       T, K, E);
    PF_HIP(hipGetLastError());
  }
}

void moe_route_counts(pfhip_backend* b, const int32_t* idx, const int32_t* counts, int tile_rows, int T, int K, int E,
                      const MoePlan& m) {
  PF_CHECK(E >= 1 && E <= 256 && K >= 1 && K <= MAXK, "moe_route_counts: need E <= 256 and K <= 8");
  PF_CHECK(tile_rows >= 1 && RBLK % tile_rows == 0, "moe_route_counts: the count tiles must divide 1024 rows");
  PF_CHECK(counts, "moe_route_counts: null counts");
  if (T <= 0) return;
  const int nblk = (T + RBLK - 1) / RBLK, n_ct = (T + tile_rows - 1) / tile_rows;
  ProfScope ps(b, "moe_route");
  hipLaunchKernelGGL(k_moe_route_counts, dim3(nblk), dim3(RBLK), 0, b->stream, idx, counts, n_ct, RBLK / tile_rows,
                     m.expert_off, m.slot_token, m.slot_of, m.tiles, m.num_tiles, T, K, E, m.tile_t);
  PF_HIP(hipGetLastError());
}

void moe_combine(pfhip_backend* b, const int32_t* idx, const float* w, const int32_t* slot_of, const void* y,
                 bool y16, const uint16_t* residual, uint16_t* moe_out, uint16_t* h_out, int T, int K, int D) {
  PF_CHECK(D > 0 && D % 4 == 0 && D <= 256 * MAXJ && K >= 1 && K <= MAXK, "moe_combine: shape out of range");
  if (T <= 0) return;
  ProfScope ps(b, "moe_combine");
  launch_combine<-1>(b, idx, w, slot_of, y, y16, residual, moe_out, h_out, nullptr, nullptr, nullptr, T, K, D, 0.0f);
}

void moe_combine_norm(pfhip_backend* b, const int32_t* idx, const float* w, const int32_t* slot_of, const void* y,
                      bool y16, const uint16_t* residual, uint16_t* h_out, const uint16_t* gamma, uint16_t* norm_hi,
                      uint16_t* norm_lo, int T, int K, int D, float eps) {
  PF_CHECK(D > 0 && D % 4 == 0 && D <= 256 * MAXJ && K >= 1 && K <= MAXK, "moe_combine: shape out of range");
  if (T <= 0) return;
  ProfScope ps(b, "moe_combine_norm");
  if (norm_lo)
    launch_combine<OUT_SPLIT>(b, idx, w, slot_of, y, y16, residual, nullptr, h_out, gamma, norm_hi, norm_lo, T, K, D,
                              eps);
  else
    launch_combine<OUT_F16>(b, idx, w, slot_of, y, y16, residual, nullptr, h_out, gamma, norm_hi, nullptr, T, K, D,
                            eps);
}

void transpose_f16(pfhip_backend* b, const uint16_t* src, uint16_t* dst, int rows, int cols) {
  if (rows <= 0 || cols <= 0) return;
  ProfScope ps(b, "transpose_f16");
  hipLaunchKernelGGL(k_transpose_f16, dim3((cols + 31) / 32, (rows + 31) / 32), dim3(256), 0, b->stream, src, dst,
                     rows, cols);
  PF_HIP(hipGetLastError());
}

void router_f16w(pfhip_backend* b, const uint16_t* x, const uint16_t* w, const uint16_t* bias, float* logits, int T,
                 int D, int E, uint16_t* wt) {
  PF_CHECK(D > 0 && D % 32 == 0 && E > 0, "router_f16w: D must be a positive multiple of 32");
  PF_CHECK(((uintptr_t)x & 15) == 0 && ((uintptr_t)wt & 15) == 0, "router_f16w: 16-byte aligned x and scratch");
  if (T <= 0) return;
  ProfScope ps(b, "router_f16w");
  hipLaunchKernelGGL(k_transpose_f16, dim3((E + 31) / 32, (D + 31) / 32), dim3(256), 0, b->stream, w, wt, D, E);
  PF_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_router_f16w, dim3((T + 15) / 16, (E + 31) / 32), dim3(64), 0, b->stream, x, wt, bias,
                     logits, T, D, E);
  PF_HIP(hipGetLastError());
}

void qmoe_gate_up_ref(pfhip_backend* b, const float* x, const int32_t* ridx, const uint8_t* w, const uint16_t* ws,
                      const uint8_t* wz, const uint16_t* bias, float* out, int T, int K, int N, int D) {
  PF_CHECK(D % 32 == 0, "qmoe_gate_up: D % 32");
  if (T * K <= 0) return;
  ProfScope ps(b, "qmoe_gate_up");
  hipLaunchKernelGGL(k_qmoe_gate_up, dim3(T * K, (N + 63) / 64), dim3(64), 0, b->stream, x, ridx, w, ws, wz, bias,
                     out, T, K, N, D);
  PF_HIP(hipGetLastError());
}

void qmoe_down_scatter_ref(pfhip_backend* b, const float* glu, const int32_t* ridx, const float* rw,
                           const uint8_t* w, const uint16_t* ws, const uint8_t* wz, const uint16_t* bias, float* acc,
                           int T, int K, int N, int D) {
  PF_CHECK(D % 32 == 0, "qmoe_down_scatter: D % 32");
  if (T <= 0) return;
  ProfScope ps(b, "qmoe_down_scatter");
  hipLaunchKernelGGL(k_qmoe_down, dim3(T, (N + 63) / 64), dim3(64), 0, b->stream, glu, ridx, rw, w, ws, wz, bias,
                     acc, T, K, N, D);
  PF_HIP(hipGetLastError());
}

}  // namespace pf
