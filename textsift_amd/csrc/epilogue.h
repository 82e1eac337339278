// epilogue.h — output stage shared by the int4 GEMM kernels.
//
// A lane holds 4 consecutive output columns n..n+3 of one output row (the
// GEMMs are computed transposed). The split numerics' conversions to fp16
// follow the WASM path (zig/math.zig:45-82) bit for bit; the cheap hardware
// conversion is used where the two agree (f16_plain) and the exact software
// path only for lanes where they may not. The fp16 numerics use the
// `_native` forms: the hardware conversions and fp16 arithmetic the
// reference's GPU shaders perform.
#pragma once
#include "common.h"
#include "pfhip_internal.h"

namespace pf {

typedef float f2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u2_t pack4(const uint16_t hb[4]) {
  return u2_t{(uint32_t)hb[0] | ((uint32_t)hb[1] << 16), (uint32_t)hb[2] | ((uint32_t)hb[3] << 16)};
}

// The exact (software) conversions, for the rare lanes the fast paths below
// cannot take. Not inlined, so the epilogues that call them stay small
// enough to unroll (their accumulators then stay in registers).
__device__ __noinline__ u2_t to_f16x4_exact(f4_t v) {
  uint16_t hb[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) hb[r] = wasm_f2h(v[r]);
  return pack4(hb);
}

// rope_apply (zig/wasm_exports.zig:1460-1502) on one pair of fp16 values:
// each product rounded to fp16, combined in f32, rounded again. c and s are
// the table entries widened as the reference widens them. Both factors of
// every product are fp16 values (<= 11 significant bits), so the product is
// exact in f32 and rounding it once to fp16 (as v_fma_mixlo_f16 does when the
// compiler fuses the conversion) equals rounding it to f32 first.
__device__ __forceinline__ void rope_pair_exact(uint16_t& ha, uint16_t& hb, float c, float s) {
  const float a = wasm_h2f(ha), b = wasm_h2f(hb);
  const float ac = wasm_h2f(wasm_f2h(a * c)), bs = wasm_h2f(wasm_f2h(b * s));
  const float bc = wasm_h2f(wasm_f2h(b * c)), as_ = wasm_h2f(wasm_f2h(a * s));
  ha = wasm_f2h(ac - bs);
  hb = wasm_f2h(bc + as_);
}

__device__ __noinline__ u2_t rope_f16x4_exact(f4_t v, f2_t cs, f2_t sn) {
  uint16_t hb[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) hb[r] = wasm_f2h(v[r]);
  rope_pair_exact(hb[0], hb[1], cs[0], sn[0]);
  rope_pair_exact(hb[2], hb[3], cs[1], sn[1]);
  return pack4(hb);
}

// 4 f32 -> 4 fp16 as wasm_f2h rounds. Where every |v| lies in
// [2^-14, 65504] both round to nearest even and the hardware packed
// conversion is used (one min/max test over the four values); otherwise
// (zeros included) the exact software path.
__device__ __forceinline__ u2_t to_f16x4(const float v[4]) {
  const float lo = fminf(fminf(fabsf(v[0]), fabsf(v[1])), fminf(fabsf(v[2]), fabsf(v[3])));
  const float hi = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  // NaN anywhere makes both comparisons false
  if (!(lo >= 6.103515625e-05f && hi <= 65504.0f)) return to_f16x4_exact(f4_t{v[0], v[1], v[2], v[3]});
  const h2_t a = __builtin_convertvector(f2_t{f32_fence(v[0]), f32_fence(v[1])}, h2_t);
  const h2_t b = __builtin_convertvector(f2_t{f32_fence(v[2]), f32_fence(v[3])}, h2_t);
  return u2_t{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
}

// to_f16x4 for data where exact zeros are common (the embedding's q == zp
// values): zeros convert to zero on both paths, so only the nonzero
// magnitudes are tested (and NaNs explicitly, which fminf / fmaxf skip).
__device__ __forceinline__ u2_t to_f16x4_z(const float v[4]) {
  float lo = 1.0f, hi = 0.0f;
  bool nan = false;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float a = fabsf(v[r]);
    lo = fminf(lo, a == 0.0f ? 1.0f : a);
    hi = fmaxf(hi, a);
    nan = nan | (v[r] != v[r]);
  }
  if (nan || !(lo >= 6.103515625e-05f && hi <= 65504.0f)) return to_f16x4_exact(f4_t{v[0], v[1], v[2], v[3]});
  const h2_t a = __builtin_convertvector(f2_t{f32_fence(v[0]), f32_fence(v[1])}, h2_t);
  const h2_t b = __builtin_convertvector(f2_t{f32_fence(v[2]), f32_fence(v[3])}, h2_t);
  return u2_t{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
}

// fp16 output of v with the RoPE rotation of pairs (n, n+1), (n+2, n+3)
// (cs, sn: the two pairs' table entries at the row's sequence position).
// The fast path needs every value that gets rounded to fp16 to lie in
// [2^-14, 65504] in magnitude (a stricter test than f16_plain: exact zeros,
// rare here, also take the exact path); one min/max over all 16 of them.
__device__ __forceinline__ u2_t rope_f16x4(const float v[4], f2_t cs, f2_t sn) {
  uint16_t hb[4];
  float lo = fminf(fminf(fabsf(v[0]), fabsf(v[1])), fminf(fabsf(v[2]), fabsf(v[3])));
  float hi = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float a = round16(v[2 * h]), b = round16(v[2 * h + 1]);
    const float c = cs[h], s = sn[h];
    const float p1 = a * c, p2 = b * s, p3 = b * c, p4 = a * s;
    lo = fminf(lo, fminf(fminf(fabsf(p1), fabsf(p2)), fminf(fabsf(p3), fabsf(p4))));
    hi = fmaxf(hi, fmaxf(fmaxf(fabsf(p1), fabsf(p2)), fmaxf(fabsf(p3), fabsf(p4))));
    const float r0 = round16_exact(p1) - round16_exact(p2);  // fp16 x fp16: exact products
    const float r1 = round16_exact(p3) + round16_exact(p4);
    lo = fminf(lo, fminf(fabsf(r0), fabsf(r1)));
    hi = fmaxf(hi, fmaxf(fabsf(r0), fabsf(r1)));
    hb[2 * h] = hw_f2h(r0);
    hb[2 * h + 1] = hw_f2h(r1);
  }
  // NaN anywhere makes both comparisons false
  if (!(lo >= 6.103515625e-05f && hi <= 65504.0f)) return rope_f16x4_exact(f4_t{v[0], v[1], v[2], v[3]}, cs, sn);
  return pack4(hb);
}

// RoPE as the reference's GPU shader computes it (native/shaders/
// rope_apply.wgsl:26-36): the GEMM result rounded to fp16, then fp16
// arithmetic throughout, each product and the sum rounded to fp16
// (v_pk_mul_f16 / v_pk_add_f16, round to nearest even, fp16 subnormals
// kept). t = {cos, sin} of pair (n, n+1), then of pair (n+2, n+3), as fp16.
// For normal fp16 values this equals the three-rounding WASM form bit for
// bit (f32 carries more than 2 x 11 + 2 bits, so rounding a difference of
// two fp16 values to f32 and then to fp16 equals rounding it once); the two
// differ only where a product or result is subnormal, which the WASM
// helpers flush to zero.
__device__ __forceinline__ u2_t rope_f16x4_native(const float v[4], h4_t t) {
  const h2_t x[2] = {__builtin_convertvector(f2_t{f32_fence(v[0]), f32_fence(v[1])}, h2_t),
                     __builtin_convertvector(f2_t{f32_fence(v[2]), f32_fence(v[3])}, h2_t)};
  uint32_t out[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const _Float16 c = t[2 * h], s = t[2 * h + 1];
    const h2_t p = x[h] * h2_t{c, c};                  // {a c, b c}
    const h2_t q = h2_t{x[h][1], x[h][0]} * h2_t{s, s};  // {b s, a s}
    out[h] = __builtin_bit_cast(uint32_t, p + h2_t{-q[0], q[1]});
  }
  return u2_t{out[0], out[1]};
}

// Stores 4 packed fp16 values at out[orow][n..n+3] (columns past N dropped).
__device__ __forceinline__ void store_f16x4(const GemmArgs& p, size_t orow, int n, u2_t hv) {
  if (p.out_f32w) {
    float* of = p.out_f32w + orow * p.ldo + n;
    const uint32_t w2[2] = {hv.x, hv.y};
    for (int r = 0; r < 4; ++r)
      if (n + r < p.N) of[r] = hw_h2f((uint16_t)(w2[r >> 1] >> (16 * (r & 1))));
    if (!p.out) return;
  }
  uint16_t* o = static_cast<uint16_t*>(p.out) + orow * p.ldo + n;
  if (n + 3 < p.N) {
    *reinterpret_cast<u2_t*>(o) = hv;
  } else {
    const uint32_t w2[2] = {hv.x, hv.y};
    for (int r = 0; r < 4; ++r)
      if (n + r < p.N) o[r] = (uint16_t)(w2[r >> 1] >> (16 * (r & 1)));
  }
}

// SWIGLU_F16 of one lane's (gate, up) column pairs (n, n+1), (n+2, n+3):
// two fp16 values packed, rounded as wasm_f2h rounds. The clamps bound every
// output to |g| <= 8 * 7, so only the low end of the fp16 range (zero and
// subnormal results, NaN) can need the exact software rounding.
__device__ __forceinline__ uint32_t swiglu_f16x2(const float v[4]) {
  const float g0 = swiglu_clamp_hw(v[0], v[1]);
  const float g1 = swiglu_clamp_hw(v[2], v[3]);
  if (!(fabsf(g0) >= 6.103515625e-05f && fabsf(g1) >= 6.103515625e-05f))
    return to_f16x4_exact(f4_t{g0, g1, 0.f, 0.f}).x;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{f32_fence(g0), f32_fence(g1)}, h2_t));
}

// The conversions of the GPU shaders' fp16 stores (hardware round to
// nearest even, fp16 subnormals kept), used by the fp16 numerics. They
// differ from wasm_f2h only for results below 2^-14 in magnitude (which the
// WASM helpers flush to zero) and in NaN payloads.
__device__ __forceinline__ u2_t to_f16x4_native(const float v[4]) {
  const h2_t a = __builtin_convertvector(f2_t{f32_fence(v[0]), f32_fence(v[1])}, h2_t);
  const h2_t b = __builtin_convertvector(f2_t{f32_fence(v[2]), f32_fence(v[3])}, h2_t);
  return u2_t{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
}
template <bool SETTLED = false>
__device__ __forceinline__ uint32_t swiglu_f16x2_native(const float v[4]) {
  const float g0 = swiglu_clamp_hw<SETTLED>(v[0], v[1]);
  const float g1 = swiglu_clamp_hw<SETTLED>(v[2], v[3]);
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{f32_fence(g0), f32_fence(g1)}, h2_t));
}

// Writes v (bias already added) for output row orow, columns n..n+3.
//   F32 / F16: out[orow][n..n+3]
//   ROPE_F16: fp16 with RoPE on columns below rope_cols (head_dim 64);
//             pos = orow % seq_len (the row's position in its sequence)
//   SWIGLU_*: (gate, up) interleaved columns -> out[orow][n/2 .. n/2+1]
template <Epi EPI>
__device__ __forceinline__ void store_out(const GemmArgs& p, size_t orow, int n, const float v[4], int pos = 0) {
  if constexpr (EPI == Epi::F32) {
    float* o = static_cast<float*>(p.out) + orow * p.ldo + n;
    if (n + 3 < p.N) {
      *reinterpret_cast<f4_t*>(o) = f4_t{v[0], v[1], v[2], v[3]};
    } else {
      for (int r = 0; r < 4; ++r)
        if (n + r < p.N) o[r] = v[r];
    }
  } else if constexpr (EPI == Epi::F16 || EPI == Epi::ROPE_F16) {
    u2_t hv;
    if constexpr (EPI == Epi::ROPE_F16) {
      if (n < p.rope_cols) {
        const int pidx = (n & 63) >> 1;
        const f2_t cs = *reinterpret_cast<const f2_t*>(p.rope_cos + pos * 32 + pidx);
        const f2_t sn = *reinterpret_cast<const f2_t*>(p.rope_sin + pos * 32 + pidx);
        hv = rope_f16x4(v, cs, sn);
      } else {
        hv = to_f16x4(v);
      }
    } else {
      hv = to_f16x4(v);
    }
    store_f16x4(p, orow, n, hv);
  } else {
    // SWIGLU_SPLIT carries the f32 result (the WASM path's numerics);
    // SWIGLU_F16 rounds it to fp16 (the GPU paths')
    const size_t oc = (size_t)(n >> 1);
    if constexpr (EPI == Epi::SWIGLU_SPLIT) {
      // f32 SwiGLU output (expert.ts keeps it f32) as hi/lo fp16 planes
      const float g0 = swiglu_clamp_fast(v[0], v[1]);
      const float g1 = swiglu_clamp_fast(v[2], v[3]);
      uint16_t a0, a1, e0, e1;
      split_hilo(g0, a0, e0);
      split_hilo(g1, a1, e1);
      *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.out) + orow * p.ldo + oc) =
          (uint32_t)a0 | ((uint32_t)a1 << 16);
      *reinterpret_cast<uint32_t*>(p.out_lo + orow * p.ldo + oc) = (uint32_t)e0 | ((uint32_t)e1 << 16);
    } else {
      *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.out) + orow * p.ldo + oc) = swiglu_f16x2(v);
    }
  }
}

}  // namespace pf
