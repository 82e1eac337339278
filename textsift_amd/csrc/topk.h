// topk.h — the reference's router top-k (topk_partial_f32,
// packages/textsift/src/zig/wasm_exports.zig:367-426) and the softmax over
// the K selected logits (softmax_f32 :919-958), shared by the stand-alone
// top-k kernel and the router GEMM's fused epilogue.
#pragma once
#include "common.h"

namespace pf {

// The reference's insertion top-k of one row, sequentially: the first K
// values sorted (an equal value never moves ahead of an earlier one), then
// each later value that beats the K-th replaces it and bubbles up. Without
// NaNs the result is the K largest values ordered by (value descending,
// index ascending); NaN comparisons short-circuit exactly as in the
// reference. x(c) returns logit c.
template <int K, typename Row>
__device__ void topk_insertion(Row x, int E, float* V, int* I) {
  for (int i = 0; i < K; ++i) { I[i] = i; V[i] = x(i); }
  for (int s = 1; s < K; ++s)
    for (int j = s; j > 0 && V[j] > V[j - 1]; --j) {
      float tv = V[j]; V[j] = V[j - 1]; V[j - 1] = tv;
      int ti = I[j]; I[j] = I[j - 1]; I[j - 1] = ti;
    }
  for (int c = K; c < E; ++c) {
    const float v = x(c);
    if (v > V[K - 1]) {
      V[K - 1] = v;
      I[K - 1] = c;
      for (int j = K - 1; j > 0 && V[j] > V[j - 1]; --j) {
        float tv = V[j]; V[j] = V[j - 1]; V[j - 1] = tv;
        int ti = I[j]; I[j] = I[j - 1]; I[j - 1] = ti;
      }
    }
  }
}

// Branch-free form for short segments: a logit and its index as one 64-bit
// key, larger = earlier in the insertion order (value descending, then
// index ascending; -0 and +0 compare equal there, so -0 is keyed as +0).
// Keys of distinct indices are distinct. Only for rows without NaNs.
__device__ __forceinline__ uint64_t topk_key(float v, int idx) {
  const uint32_t u = __float_as_uint(v + 0.0f);  // -0 -> +0
  const uint32_t o = u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);  // order-preserving
  return ((uint64_t)o << 32) | (uint32_t)(0xFFFF - idx);
}
__device__ __forceinline__ int topk_key_index(uint64_t k) { return 0xFFFF - (int)(uint32_t)(k & 0xFFFFu); }

// compare-exchange: a keeps the larger key
__device__ __forceinline__ void topk_ce(uint64_t& a, uint64_t& b) {
  const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
  a = hi;
  b = lo;
}

// four keys sorted descending
__device__ __forceinline__ void topk_sort4(uint64_t* k) {
  topk_ce(k[0], k[1]);
  topk_ce(k[2], k[3]);
  topk_ce(k[0], k[2]);
  topk_ce(k[1], k[3]);
  topk_ce(k[1], k[2]);
}

// the 4 largest of two descending lists of 4 (into a), descending: the
// pairwise maxima of a and reversed b form a bitonic sequence holding them
__device__ __forceinline__ void topk_merge4(uint64_t* a, const uint64_t* b) {
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = a[i] > b[3 - i] ? a[i] : b[3 - i];
  topk_ce(a[0], a[2]);
  topk_ce(a[1], a[3]);
  topk_ce(a[0], a[1]);
  topk_ce(a[2], a[3]);
}

// Routing weights of the K selected logits V (sorted as above): softmax
// with libm exp, times wscale; written with the expert ids to idx / w.
template <int K>
__device__ __forceinline__ void topk_write(const float* V, const int* I, float wscale, int32_t* idx, float* w) {
  float mx = V[0];
#pragma unroll
  for (int c = 1; c < K; ++c) if (V[c] > mx) mx = V[c];
  float e[K], sum = 0.0f;
#pragma unroll
  for (int c = 0; c < K; ++c) { e[c] = expf(V[c] - mx); sum += e[c]; }
  const float inv = sum > 0.0f ? 1.0f / sum : 1.0f / (float)K;
#pragma unroll
  for (int c = 0; c < K; ++c) {
    idx[c] = I[c];
    w[c] = (e[c] * inv) * wscale;
  }
}

}  // namespace pf
