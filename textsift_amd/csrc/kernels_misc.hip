// kernels_misc.hip — HBM-bound kernels of the forward: the
// GatherBlockQuantized embedding, RMSNorm variants, element-wise ops, the
// router top-k, the MoE routing plan (a deterministic counting sort) and the
// MoE combine. Reference semantics: packages/textsift/src/zig/wasm_exports.zig
// (line ranges cited per kernel).
#include "common.cuh"
#include "pfhip_internal.h"

namespace pf {

namespace {

constexpr int ROWS_PER_BLOCK = 4;  // one wave per row, 4 waves per block

// ----------------------------------------------------------------------------
// GatherBlockQuantized (embed_lookup_int4, :1523-1573): one wave per token
// row. Lane l owns 16 B of packed nibbles (32 values = one quant block) for
// lanes 0..D/32-1; the row's scales / zero-points are read once per lane.
// fp16((q - zp) * scale) is a single rounding of an exact product, so the
// output is bit-identical to the reference.
__global__ __launch_bounds__(256) void k_embed(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                               const uint8_t* __restrict__ zp, const int32_t* __restrict__ ids,
                                               uint16_t* __restrict__ out, int T, int V, int D) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (t >= T) return;
  const int nb = D >> 5;
  const int id = ids[t];
  uint16_t* o = out + (size_t)t * D;
  for (int blk = lane; blk < nb; blk += 64) {
    u4_t res[4] = {};
    if (id >= 0 && id < V) {
      const size_t row = (size_t)id;
      const u4_t w = *reinterpret_cast<const u4_t*>(q + row * (D >> 1) + blk * 16);
      const float sc = wasm_h2f(s[row * nb + blk]);
      const uint8_t zb = zp[row * ((nb + 1) >> 1) + (blk >> 1)];
      const int z = (blk & 1) ? (zb >> 4) : (zb & 0xF);
      const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int wi = 0; wi < 4; ++wi) {
        uint32_t packed[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t byte = (words[wi] >> (8 * j)) & 0xFFu;
          const float lo = (float)((int)(byte & 0xF) - z) * sc;
          const float hi = (float)((int)(byte >> 4) - z) * sc;
          packed[j] = (uint32_t)wasm_f2h(lo) | ((uint32_t)wasm_f2h(hi) << 16);
        }
        res[wi] = u4_t{packed[0], packed[1], packed[2], packed[3]};
      }
    }
    u4_t* dst = reinterpret_cast<u4_t*>(o + blk * 32);
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) dst[wi] = res[wi];
  }
}

// ----------------------------------------------------------------------------
// RMSNorm family (:186-350). One wave per row, the row held in registers
// (D <= 64 * 16). Widening is the reference's bit trick (wasm_h2f).
constexpr int MAXPL = 16;  // elements per lane

// Output forms of a normalised row: fp16, f32, or the f32 value as hi/lo fp16 planes.
enum OutMode { OUT_F16 = 0, OUT_F32 = 1, OUT_SPLIT = 2 };

template <int MODE>
__device__ __forceinline__ void put(void* out, uint16_t* out_lo, size_t i, float y) {
  if constexpr (MODE == OUT_F32) {
    static_cast<float*>(out)[i] = y;
  } else if constexpr (MODE == OUT_F16) {
    static_cast<uint16_t*>(out)[i] = wasm_f2h(y);
  } else {
    uint16_t h, l;
    split_hilo(y, h, l);
    static_cast<uint16_t*>(out)[i] = h;
    out_lo[i] = l;
  }
}

template <int MODE>
__global__ __launch_bounds__(256) void k_rms_norm(const uint16_t* __restrict__ x, const uint16_t* __restrict__ g,
                                                  void* __restrict__ out, uint16_t* __restrict__ out_lo, int T, int D,
                                                  float eps) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (t >= T) return;
  const uint16_t* xr = x + (size_t)t * D;
  float v[MAXPL];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < MAXPL; ++i) {
    const int d = i * 64 + lane;
    v[i] = d < D ? wasm_h2f(xr[d]) : 0.0f;
    ss += v[i] * v[i];
  }
  ss = wave_sum(ss);
  const float d_inv = 1.0f / (float)D;
  const float inv_rms = 1.0f / sqrtf(ss * d_inv + eps);
#pragma unroll
  for (int i = 0; i < MAXPL; ++i) {
    const int d = i * 64 + lane;
    if (d < D) put<MODE>(out, out_lo, (size_t)t * D + d, v[i] * inv_rms * wasm_h2f(g[d]));
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
  uint16_t hs[MAXPL];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < MAXPL; ++i) {
    const int d = i * 64 + lane;
    float sv = 0.0f;
    if (d < D) {
      sv = wasm_h2f(a[base + d]) + wasm_h2f(bb[base + d]);
      hs[i] = wasm_f2h(sv);
      sum_out[base + d] = hs[i];
    }
    ss += sv * sv;
  }
  ss = wave_sum(ss);
  const float inv_rms = 1.0f / sqrtf(ss * (1.0f / (float)D) + eps);
#pragma unroll
  for (int i = 0; i < MAXPL; ++i) {
    const int d = i * 64 + lane;
    if (d < D) put<MODE>(norm_out, norm_lo, base + d, wasm_h2f(hs[i]) * inv_rms * wasm_h2f(g[d]));
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
// Router top-k + softmax (topk_partial_f32 :367-426, softmax_f32 :919-958).
// One thread per token replays the reference's insertion order exactly:
// output sorted by logit descending, ties keep the lower expert id first.
constexpr int MAXK = 8;
__global__ __launch_bounds__(256) void k_router_topk(const float* __restrict__ logits, int32_t* __restrict__ idx,
                                                     float* __restrict__ w, int T, int E, int K, float wscale) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const float* x = logits + (size_t)t * E;
  float V[MAXK];
  int I[MAXK];
  for (int i = 0; i < K; ++i) { I[i] = i; V[i] = x[i]; }
  for (int s = 1; s < K; ++s)
    for (int j = s; j > 0 && V[j] > V[j - 1]; --j) {
      float tv = V[j]; V[j] = V[j - 1]; V[j - 1] = tv;
      int ti = I[j]; I[j] = I[j - 1]; I[j - 1] = ti;
    }
  for (int c = K; c < E; ++c) {
    const float v = x[c];
    if (v > V[K - 1]) {
      V[K - 1] = v;
      I[K - 1] = c;
      for (int j = K - 1; j > 0 && V[j] > V[j - 1]; --j) {
        float tv = V[j]; V[j] = V[j - 1]; V[j - 1] = tv;
        int ti = I[j]; I[j] = I[j - 1]; I[j - 1] = ti;
      }
    }
  }
  float mx = V[0];
  for (int c = 1; c < K; ++c) if (V[c] > mx) mx = V[c];
  float e[MAXK], sum = 0.0f;
  for (int c = 0; c < K; ++c) { e[c] = expf(V[c] - mx); sum += e[c]; }
  const float inv = sum > 0.0f ? 1.0f / sum : 1.0f / (float)K;
  for (int c = 0; c < K; ++c) {
    idx[(size_t)t * K + c] = I[c];
    w[(size_t)t * K + c] = (e[c] * inv) * wscale;
  }
}

// ----------------------------------------------------------------------------
// MoE routing plan: a stable counting sort of the T*K (token, k) pairs by
// expert, reproducing the reference's per-expert lists (for e ascending, the
// pairs with expert e in ascending token order: browser/inference/
// expert.ts:125-145). Deterministic: no atomics anywhere.
constexpr int RBLK = 256;  // tokens per counting block

// counts[blk][e] = occurrences of e among the block's tokens. Thread e scans
// the block's routing rows from LDS (broadcast reads).
__global__ __launch_bounds__(256) void k_moe_count(const int32_t* __restrict__ idx, int32_t* __restrict__ counts,
                                                   int T, int K, int E) {
  __shared__ int32_t sidx[RBLK * MAXK];
  const int blk = blockIdx.x;
  const int t0 = blk * RBLK;
  const int nt = min(RBLK, T - t0);
  for (int i = threadIdx.x; i < nt * K; i += blockDim.x) sidx[i] = idx[(size_t)t0 * K + i];
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int c = 0;
    for (int i = 0; i < nt * K; ++i) c += sidx[i] == e;
    counts[(size_t)blk * E + e] = c;
  }
}

// Single workgroup: expert offsets, per-(block, expert) offsets and the
// grouped-GEMM tile list (expert, row0, rows).
__global__ __launch_bounds__(256) void k_moe_scan(const int32_t* __restrict__ counts, int32_t* __restrict__ blk_off,
                                                  int32_t* __restrict__ expert_off, int32_t* __restrict__ tiles,
                                                  int32_t* __restrict__ num_tiles, int nblk, int E, int tile_t) {
  __shared__ int32_t tot[256];
  __shared__ int32_t ntl[256];
  const int e = threadIdx.x;
  int total = 0;
  if (e < E)
    for (int b = 0; b < nblk; ++b) total += counts[(size_t)b * E + e];
  tot[e] = e < E ? total : 0;
  ntl[e] = e < E ? (total + tile_t - 1) / tile_t : 0;
  __syncthreads();
  if (e == 0) {  // sequential exclusive scans over <= 256 experts
    int acc = 0, tacc = 0;
    for (int i = 0; i < E; ++i) {
      const int c = tot[i], n = ntl[i];
      tot[i] = acc;
      ntl[i] = tacc;
      acc += c;
      tacc += n;
    }
    expert_off[E] = acc;
    *num_tiles = tacc;
  }
  __syncthreads();
  if (e < E) {
    const int base = tot[e];
    expert_off[e] = base;
    int run = base;
    for (int b = 0; b < nblk; ++b) {
      blk_off[(size_t)b * E + e] = run;
      run += counts[(size_t)b * E + e];
    }
    int tix = ntl[e];
    for (int r = 0; r < total; r += tile_t, ++tix) {
      tiles[tix * 4 + 0] = e;
      tiles[tix * 4 + 1] = base + r;
      tiles[tix * 4 + 2] = min(tile_t, total - r);
      tiles[tix * 4 + 3] = 0;
    }
  }
}

// Slot assignment: thread e walks the block's tokens in order.
__global__ __launch_bounds__(256) void k_moe_scatter(const int32_t* __restrict__ idx,
                                                     const int32_t* __restrict__ blk_off,
                                                     int32_t* __restrict__ slot_token, int32_t* __restrict__ slot_of,
                                                     int T, int K, int E) {
  __shared__ int32_t sidx[RBLK * MAXK];
  const int blk = blockIdx.x;
  const int t0 = blk * RBLK;
  const int nt = min(RBLK, T - t0);
  for (int i = threadIdx.x; i < nt * K; i += blockDim.x) sidx[i] = idx[(size_t)t0 * K + i];
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int pos = blk_off[(size_t)blk * E + e];
    for (int i = 0; i < nt * K; ++i)
      if (sidx[i] == e) {
        slot_token[pos] = t0 + i / K;
        slot_of[(size_t)t0 * K + i] = pos;
        ++pos;
      }
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
template <int NMODE>
__global__ __launch_bounds__(256) void k_moe_combine(const int32_t* __restrict__ idx, const float* __restrict__ w,
                                                     const int32_t* __restrict__ slot_of, const float* __restrict__ y,
                                                     const uint16_t* __restrict__ residual,
                                                     uint16_t* __restrict__ moe_out, uint16_t* __restrict__ h_out,
                                                     const uint16_t* __restrict__ gamma,
                                                     uint16_t* __restrict__ norm_hi, uint16_t* __restrict__ norm_lo,
                                                     int T, int K, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (t >= T) return;
  int ek[MAXK], sk[MAXK];
  float wk[MAXK];
  for (int k = 0; k < K; ++k) {
    ek[k] = idx[(size_t)t * K + k];
    wk[k] = w[(size_t)t * K + k];
    sk[k] = slot_of[(size_t)t * K + k];
  }
  for (int a = 1; a < K; ++a)  // insertion sort by expert id (ids are distinct)
    for (int j = a; j > 0 && ek[j] < ek[j - 1]; --j) {
      int te = ek[j]; ek[j] = ek[j - 1]; ek[j - 1] = te;
      float tw = wk[j]; wk[j] = wk[j - 1]; wk[j - 1] = tw;
      int ts = sk[j]; sk[j] = sk[j - 1]; sk[j - 1] = ts;
    }
  const size_t base = (size_t)t * D;
  uint16_t hs[MAXPL];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < MAXPL; ++i) {
    const int d = i * 64 + lane;
    float hv = 0.0f;
    if (d < D) {
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) acc = fmaf(wk[k], y[(size_t)sk[k] * D + d], acc);
      const uint16_t m = wasm_f2h(acc);
      if (moe_out) moe_out[base + d] = m;
      hs[i] = wasm_f2h(wasm_h2f(residual[base + d]) + wasm_h2f(m));
      h_out[base + d] = hs[i];
      hv = wasm_h2f(hs[i]);
    }
    ss += hv * hv;
  }
  if constexpr (NMODE >= 0) {
    // the next block's rms_norm_fp16_to_f32 on the new residual row (:220-270)
    ss = wave_sum(ss);
    const float inv_rms = 1.0f / sqrtf(ss * (1.0f / (float)D) + eps);
#pragma unroll
    for (int i = 0; i < MAXPL; ++i) {
      const int d = i * 64 + lane;
      if (d < D) put<NMODE>(norm_hi, norm_lo, base + d, wasm_h2f(hs[i]) * inv_rms * wasm_h2f(gamma[d]));
    }
  }
}

// ----------------------------------------------------------------------------
// fp16-weight router (router W fp16 [D][E], f32 accumulate,
// bias fp16): logits[t][e] = sum_d x[t][d] W[d][e] + bias[e]. One thread per
// (t, e); 4-lane partial sums combined as the reference's TR=8 path does.
__global__ __launch_bounds__(128) void k_router_f16w(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                     const uint16_t* __restrict__ bias, float* __restrict__ logits,
                                                     int T, int D, int E) {
  extern __shared__ float xs[];
  const int t = blockIdx.x;
  for (int d = threadIdx.x; d < D; d += blockDim.x) xs[d] = wasm_h2f(x[(size_t)t * D + d]);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    float l[4] = {0.f, 0.f, 0.f, 0.f};
    int d = 0;
    for (; d + 4 <= D; d += 4)
#pragma unroll
      for (int c = 0; c < 4; ++c) l[c] = fmaf(xs[d + c], wasm_h2f(w[(size_t)(d + c) * E + e]), l[c]);
    float s = (l[0] + l[1]) + (l[2] + l[3]);
    for (; d < D; ++d) s = fmaf(xs[d], wasm_h2f(w[(size_t)d * E + e]), s);
    logits[(size_t)t * E + e] = s + (bias ? wasm_h2f(bias[e]) : 0.0f);
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

}  // namespace

void embed_lookup(pfhip_backend* b, const uint8_t* q, const uint16_t* s, const uint8_t* zp, const int32_t* ids,
                  uint16_t* out, int T, int V, int D) {
  PF_CHECK(D % 32 == 0 && D / 32 <= 64 * 4, "embed_lookup: D must be a multiple of 32");
  PF_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)out & 15) == 0 && (D / 2) % 16 == 0,
           "embed_lookup: table and output must be 16-byte aligned");
  if (T <= 0) return;
  ProfScope ps(b, "embed_lookup_int4");
  hipLaunchKernelGGL(k_embed, dim3((T + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK), dim3(256), 0, b->stream, q, s, zp,
                     ids, out, T, V, D);
  PF_HIP(hipGetLastError());
}

void rms_norm_f16(pfhip_backend* b, const uint16_t* x, const uint16_t* g, uint16_t* out, int T, int D, float eps) {
  PF_CHECK(D > 0 && D <= 64 * MAXPL, "rms_norm: D out of range");
  if (T <= 0) return;
  ProfScope ps(b, "rms_norm");
  hipLaunchKernelGGL(k_rms_norm<OUT_F16>, dim3((T + 3) / 4), dim3(256), 0, b->stream, x, g, out, nullptr, T, D, eps);
  PF_HIP(hipGetLastError());
}

void rms_norm_f32(pfhip_backend* b, const uint16_t* x, const uint16_t* g, float* out, int T, int D, float eps) {
  PF_CHECK(D > 0 && D <= 64 * MAXPL, "rms_norm: D out of range");
  if (T <= 0) return;
  ProfScope ps(b, "rms_norm_fp16_to_f32");
  hipLaunchKernelGGL(k_rms_norm<OUT_F32>, dim3((T + 3) / 4), dim3(256), 0, b->stream, x, g, out, nullptr, T, D, eps);
  PF_HIP(hipGetLastError());
}

void rms_norm_split(pfhip_backend* b, const uint16_t* x, const uint16_t* g, uint16_t* hi, uint16_t* lo, int T, int D,
                    float eps) {
  PF_CHECK(D > 0 && D <= 64 * MAXPL, "rms_norm: D out of range");
  if (T <= 0) return;
  ProfScope ps(b, "rms_norm_split");
  hipLaunchKernelGGL(k_rms_norm<OUT_SPLIT>, dim3((T + 3) / 4), dim3(256), 0, b->stream, x, g, hi, lo, T, D, eps);
  PF_HIP(hipGetLastError());
}

void add_rms_norm_f32(pfhip_backend* b, const uint16_t* a, const uint16_t* bb, const uint16_t* g, uint16_t* sum_out,
                      float* norm_out, int T, int D, float eps) {
  PF_CHECK(D > 0 && D <= 64 * MAXPL, "add_rmsnorm: D out of range");
  if (T <= 0) return;
  ProfScope ps(b, "add_rmsnorm_fp16_to_f32");
  hipLaunchKernelGGL(k_add_rms_norm<OUT_F32>, dim3((T + 3) / 4), dim3(256), 0, b->stream, a, bb, g, sum_out,
                     norm_out, nullptr, T, D, eps);
  PF_HIP(hipGetLastError());
}

void add_rms_norm_f16(pfhip_backend* b, const uint16_t* a, const uint16_t* bb, const uint16_t* g, uint16_t* sum_out,
                      uint16_t* norm_out, int T, int D, float eps) {
  PF_CHECK(D > 0 && D <= 64 * MAXPL, "add_rmsnorm: D out of range");
  if (T <= 0) return;
  ProfScope ps(b, "add_rmsnorm_f16");
  hipLaunchKernelGGL(k_add_rms_norm<OUT_F16>, dim3((T + 3) / 4), dim3(256), 0, b->stream, a, bb, g, sum_out,
                     norm_out, nullptr, T, D, eps);
  PF_HIP(hipGetLastError());
}

void add_rms_norm_split(pfhip_backend* b, const uint16_t* a, const uint16_t* bb, const uint16_t* g,
                        uint16_t* sum_out, uint16_t* hi, uint16_t* lo, int T, int D, float eps) {
  PF_CHECK(D > 0 && D <= 64 * MAXPL, "add_rmsnorm: D out of range");
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
  ProfScope ps(b, "router_topk");
  hipLaunchKernelGGL(k_router_topk, dim3((T + 255) / 256), dim3(256), 0, b->stream, logits, idx, w, T, E, K, wscale);
  PF_HIP(hipGetLastError());
}

int moe_max_tiles(int T, int K, int E, int tile_t) { return (T * K + tile_t - 1) / tile_t + E; }

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t moe_plan_bytes(int T, int K, int E, int tile_t) {
  const size_t nblk = (size_t)(T + RBLK - 1) / RBLK;
  return al256(nblk * E * 4) * 2 + al256((size_t)(E + 1) * 4) + al256((size_t)T * K * 4) * 2 +
         al256((size_t)moe_max_tiles(T, K, E, tile_t) * 16) + 256;
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
  m.num_tiles = reinterpret_cast<int32_t*>(p);
  m.max_tiles = moe_max_tiles(T, K, E, tile_t);
  m.tile_t = tile_t;
  return m;
}

void moe_route(pfhip_backend* b, const int32_t* idx, int T, int K, int E, const MoePlan& m) {
  PF_CHECK(E >= 1 && E <= 256 && K >= 1 && K <= MAXK, "moe_route: need E <= 256 and K <= 8");
  if (T <= 0) return;
  const int nblk = (T + RBLK - 1) / RBLK;
  {
    ProfScope ps(b, "moe_count");
    hipLaunchKernelGGL(k_moe_count, dim3(nblk), dim3(256), 0, b->stream, idx, m.counts, T, K, E);
    PF_HIP(hipGetLastError());
  }
  {
    ProfScope ps(b, "moe_scan");
    hipLaunchKernelGGL(k_moe_scan, dim3(1), dim3(256), 0, b->stream, m.counts, m.blk_off, m.expert_off, m.tiles,
                       m.num_tiles, nblk, E, m.tile_t);
    PF_HIP(hipGetLastError());
  }
  {
    ProfScope ps(b, "moe_scatter");
    hipLaunchKernelGGL(k_moe_scatter, dim3(nblk), dim3(256), 0, b->stream, idx, m.blk_off, m.slot_token, m.slot_of,
                       T, K, E);
    PF_HIP(hipGetLastError());
  }
}

void moe_combine(pfhip_backend* b, const int32_t* idx, const float* w, const int32_t* slot_of, const float* y,
                 const uint16_t* residual, uint16_t* moe_out, uint16_t* h_out, int T, int K, int D) {
  PF_CHECK(D <= 64 * MAXPL && K <= MAXK, "moe_combine: shape out of range");
  if (T <= 0) return;
  ProfScope ps(b, "moe_combine");
  hipLaunchKernelGGL(k_moe_combine<-1>, dim3((T + 3) / 4), dim3(256), 0, b->stream, idx, w, slot_of, y, residual,
                     moe_out, h_out, nullptr, nullptr, nullptr, T, K, D, 0.0f);
  PF_HIP(hipGetLastError());
}

void moe_combine_norm(pfhip_backend* b, const int32_t* idx, const float* w, const int32_t* slot_of, const float* y,
                      const uint16_t* residual, uint16_t* h_out, const uint16_t* gamma, uint16_t* norm_hi,
                      uint16_t* norm_lo, int T, int K, int D, float eps) {
  PF_CHECK(D <= 64 * MAXPL && K <= MAXK, "moe_combine: shape out of range");
  if (T <= 0) return;
  ProfScope ps(b, "moe_combine_norm");
  if (norm_lo)
    hipLaunchKernelGGL(k_moe_combine<OUT_SPLIT>, dim3((T + 3) / 4), dim3(256), 0, b->stream, idx, w, slot_of, y,
                       residual, nullptr, h_out, gamma, norm_hi, norm_lo, T, K, D, eps);
  else
    hipLaunchKernelGGL(k_moe_combine<OUT_F16>, dim3((T + 3) / 4), dim3(256), 0, b->stream, idx, w, slot_of, y,
                       residual, nullptr, h_out, gamma, norm_hi, nullptr, T, K, D, eps);
  PF_HIP(hipGetLastError());
}

void router_f16w(pfhip_backend* b, const uint16_t* x, const uint16_t* w, const uint16_t* bias, float* logits, int T,
                 int D, int E) {
  PF_CHECK(D > 0 && D <= 16384 && E > 0, "router_f16w: bad shape");
  if (T <= 0) return;
  ProfScope ps(b, "router_f16w");
  hipLaunchKernelGGL(k_router_f16w, dim3(T), dim3(128), D * sizeof(float), b->stream, x, w, bias, logits, T, D, E);
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
