// Device code of the MoE combine: the output forms of a normalised row and
// one token's combine (the per-token body of the combine kernel in
// kernels_misc.hip, callable from any kernel that holds a wave per token).
#pragma once

#include <type_traits>

#include "common.h"
#include "epilogue.h"

namespace pf {
namespace {

// Output forms of a normalised row: fp16, f32, or the f32 value as hi/lo fp16 planes.
enum OutMode { OUT_F16 = 0, OUT_F32 = 1, OUT_SPLIT = 2 };


__device__ __forceinline__ void h4_to_f(u2_t w, float v[4]) { h4_widen(w, v); }

template <int MODE>
__device__ __forceinline__ void put4(void* out, uint16_t* out_lo, size_t i, const float y[4]) {
  if constexpr (MODE == OUT_F32) {
    *reinterpret_cast<f4_t*>(static_cast<float*>(out) + i) = f4_t{y[0], y[1], y[2], y[3]};
  } else if constexpr (MODE == OUT_F16) {
    *reinterpret_cast<u2_t*>(static_cast<uint16_t*>(out) + i) = to_f16x4(y);
  } else {
    uint16_t h[4], l[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) split_hilo(y[r], h[r], l[r]);
    *reinterpret_cast<u2_t*>(static_cast<uint16_t*>(out) + i) = pack4(h);
    *reinterpret_cast<u2_t*>(out_lo + i) = pack4(l);
  }
}


// One token's combine (k_moe_combine in kernels_misc.hip), in three steps so
// that a wave can keep several tokens' loads in flight: comb_index (the
// token's K expert ids, routing weights and slots, sorted by ascending expert
// id), comb_load (every load of the row, issued before any is used) and
// comb_finish (sum the K expert outputs with fused multiply-adds in ascending
// expert id, add the residual, and for NMODE >= 0 the next block's RMSNorm
// of the new residual row). Lane `lane` of the token's wave holds elements
// 4 lane + 256 j .. +3. The results go to store_m(d, moe out), store_h(d,
// new residual) and store_n(d, norm values), so every caller gets the same
// bits.
template <int K>
struct CombIdx {
  int e[K], s[K];
  float w[K];
};

template <int K>
__device__ __forceinline__ CombIdx<K> comb_index(int t, const int32_t* __restrict__ idx, const float* __restrict__ w,
                                                 const int32_t* __restrict__ slot_of) {
  CombIdx<K> c;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    c.e[k] = idx[(size_t)t * K + k];
    c.w[k] = w[(size_t)t * K + k];
    c.s[k] = slot_of[(size_t)t * K + k];
  }
  // ascending expert id (ids are distinct): a fixed compare-exchange network
#pragma unroll
  for (int a = 1; a < K; ++a)
#pragma unroll
    for (int j = a; j > 0; --j) {
      const bool sw = c.e[j] < c.e[j - 1];
      const int e0 = c.e[j - 1], e1 = c.e[j], s0 = c.s[j - 1], s1 = c.s[j];
      const float w0 = c.w[j - 1], w1 = c.w[j];
      c.e[j - 1] = sw ? e1 : e0;
      c.e[j] = sw ? e0 : e1;
      c.s[j - 1] = sw ? s1 : s0;
      c.s[j] = sw ? s0 : s1;
      c.w[j - 1] = sw ? w1 : w0;
      c.w[j] = sw ? w0 : w1;
    }
  return c;
}

// the loaded operands of one token's row: expert outputs (fp16 bits with
// Y16, else f32), residual and gamma units
template <int K, int NJ, bool Y16>
struct CombRow {
  std::conditional_t<Y16, u2_t, f4_t> y[NJ][K];
  u2_t r[NJ], g[NJ];
};

template <int NMODE, int K, int NJ, bool Y16, bool RES>
__device__ __forceinline__ CombRow<K, NJ, Y16> comb_load(int t, int lane, const CombIdx<K>& c,
                                                         const void* __restrict__ y,
                                                         const uint16_t* __restrict__ residual,
                                                         const uint16_t* __restrict__ gamma, int D) {
  CombRow<K, NJ, Y16> L;
  const size_t base = (size_t)t * D;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int d = 4 * lane + 256 * j;
    if (d < D) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        if constexpr (Y16) {
          // read once: non-temporal, so the 168 MB of expert outputs do not
          // push the next GEMM's activations and weights out of the caches
          // (the QKV GEMM that follows: 68.5 -> 66 us; forward -1 %)
          L.y[j][k] = __builtin_nontemporal_load(
              reinterpret_cast<const u2_t*>(static_cast<const uint16_t*>(y) + (size_t)c.s[k] * D + d));
        } else {
          L.y[j][k] = *reinterpret_cast<const f4_t*>(static_cast<const float*>(y) + (size_t)c.s[k] * D + d);
        }
      }
      if constexpr (RES) L.r[j] = *reinterpret_cast<const u2_t*>(residual + base + d);
      else L.r[j] = u2_t{0u, 0u};
      if constexpr (NMODE >= 0) L.g[j] = *reinterpret_cast<const u2_t*>(gamma + d);
    }
  }
  return L;
}

template <int NMODE, int K, int NJ, bool Y16, class SM, class SH, class SN>
__device__ __forceinline__ void comb_finish(int lane, const CombIdx<K>& c, const CombRow<K, NJ, Y16>& L, int D,
                                            float eps, SM store_m, SH store_h, SN store_n) {
  u2_t hs[NJ];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int d = 4 * lane + 256 * j;
    hs[j] = u2_t{0u, 0u};
    if (d < D) {
      f4_t yv[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        if constexpr (Y16) {
          const h4_t h = __builtin_bit_cast(h4_t, L.y[j][k]);
          yv[k] = f4_t{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
        } else {
          yv[k] = L.y[j][k];
        }
      }
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k = 0; k < K; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(c.w[k], yv[k][r], acc[r]);
      const u2_t m = to_f16x4(acc);
      store_m(d, m);
      float mv[4], rv[4], sv[4];
      h4_to_f(m, mv);
      h4_to_f(L.r[j], rv);
#pragma unroll
      for (int r = 0; r < 4; ++r) sv[r] = rv[r] + mv[r];
      hs[j] = to_f16x4(sv);
      store_h(d, hs[j]);
      float hv[4];
      h4_to_f(hs[j], hv);
#pragma unroll
      for (int r = 0; r < 4; ++r) ss += hv[r] * hv[r];
    }
  }
  if constexpr (NMODE >= 0) {
    // the next block's rms_norm_fp16_to_f32 on the new residual row (:220-270)
    ss = wave_sum(ss);
    const float inv_rms = 1.0f / sqrtf(ss * (1.0f / (float)D) + eps);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int d = 4 * lane + 256 * j;
      if (d < D) {
        float hv[4], gm[4], yo[4];
        h4_to_f(hs[j], hv);
        h4_to_f(L.g[j], gm);
#pragma unroll
        for (int r = 0; r < 4; ++r) yo[r] = hv[r] * inv_rms * gm[r];
        store_n(d, yo);
      }
    }
  }
}

// One token's combine with its results in global memory (the combine kernel).
template <int NMODE, int K, int NJ, bool Y16, bool RES>
__device__ __forceinline__ void moe_combine_row(int t, int lane, const int32_t* __restrict__ idx,
                                                const float* __restrict__ w, const int32_t* __restrict__ slot_of,
                                                const void* __restrict__ y, const uint16_t* __restrict__ residual,
                                                uint16_t* __restrict__ moe_out, uint16_t* __restrict__ h_out,
                                                const uint16_t* __restrict__ gamma, uint16_t* __restrict__ norm_hi,
                                                uint16_t* __restrict__ norm_lo, int D, float eps) {
  const CombIdx<K> c = comb_index<K>(t, idx, w, slot_of);
  const CombRow<K, NJ, Y16> L = comb_load<NMODE, K, NJ, Y16, RES>(t, lane, c, y, residual, gamma, D);
  const size_t base = (size_t)t * D;
  comb_finish<NMODE, K, NJ, Y16>(
      lane, c, L, D, eps,
      [&](int d, u2_t m) {
        if (moe_out) *reinterpret_cast<u2_t*>(moe_out + base + d) = m;
      },
      [&](int d, u2_t hv) { *reinterpret_cast<u2_t*>(h_out + base + d) = hv; },
      [&](int d, const float* yo) { put4<NMODE>(norm_hi, norm_lo, base + d, yo); });
}

}  // namespace
}  // namespace pf
