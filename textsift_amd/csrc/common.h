// common.h — device helpers shared by the gfx950 kernels.
//
// Numerics follow the reference's WASM path
// (packages/textsift/src/zig/math.zig, zig/wasm_exports.zig): every kernel
// is compiled with -ffp-contract=off, and the places where the reference
// fuses a multiply-add (its relaxed_madd sites, c/fma.c:10-13) call fmaf()
// explicitly.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pf {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

// fp16 bits -> f32 as zig/math.zig:45-52 computes it: exact for normals and
// zero; subnormals / inf / NaN get the blind exponent rebias
// (m -> 2^-15 (1 + m/1024), inf -> 65536).
__device__ __forceinline__ float wasm_h2f(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t rest = (uint32_t)h & 0x7fffu;
  uint32_t biased = rest == 0u ? 0u : (rest << 13) + (112u << 23);
  return __uint_as_float(sign | biased);
}

// f32 -> fp16 bits as zig/math.zig:54-82: RNE for normal results (what the
// hardware conversion does), round-half-up for subnormal results.
// The compiler may fuse "round an f32 product or sum to fp16" into one
// v_fma_mix*_f16, which rounds the exact result once instead of rounding it
// to f32 first. f32_fence makes the value an opaque f32 so the conversions
// below round exactly the f32 value they are given.
__device__ __forceinline__ float f32_fence(float f) {
  asm("" : "+v"(f));
  return f;
}

__device__ __forceinline__ uint16_t wasm_f2h(float f) {
  f = f32_fence(f);
  const float a = fabsf(f);
  if (a >= 6.103515625e-05f || !(a == a)) {
    _Float16 h = (_Float16)f;
    uint16_t bits = __builtin_bit_cast(uint16_t, h);
    if (!(a == a)) bits = (uint16_t)((bits & 0x8000u) | 0x7e00u);  // NaN: quiet bit (math.zig:59)
    return bits;
  }
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t exp32 = (u >> 23) & 0xffu;
  int32_t e16 = (int32_t)exp32 - 127 + 15;
  if (e16 < -10) return (uint16_t)sign;
  uint32_t shift = (uint32_t)(14 - e16);
  uint32_t mant24 = (u & 0x7fffffu) | 0x800000u;
  return (uint16_t)(sign | ((mant24 + (1u << (shift - 1))) >> shift));
}

// True when the fp16 rounding of f involves none of the cases in which the
// wasm helpers differ from the hardware: f is zero or |f| lies in
// [2^-14, 65504] (no subnormal, overflow or NaN result). For such f,
// wasm_f2h(f) is the hardware conversion and wasm_h2f of the result is the
// hardware widening.
__device__ __forceinline__ bool f16_plain(float f) {
  const uint32_t a = __float_as_uint(f) & 0x7fffffffu;
  return a == 0u || a - 0x38800000u <= 0x0EFFE000u;
}

// Hardware f32 -> fp16 (round to nearest even) and the fp16 round trip, of
// the f32 value given (fenced, see f32_fence).
__device__ __forceinline__ uint16_t hw_f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f32_fence(f)); }
__device__ __forceinline__ float round16(float f) { return (float)(_Float16)f32_fence(f); }
// The fp16 round trip of a value the caller knows to be exact in f32 (such
// as a product of two fp16 values): a fused single rounding is then the
// same, so no fence.
__device__ __forceinline__ float round16_exact(float f) { return (float)(_Float16)f; }

// Hardware IEEE widen (used for MFMA operands; differs from wasm_h2f only on
// fp16 subnormals).
__device__ __forceinline__ float hw_h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

typedef uint16_t us2_t __attribute__((ext_vector_type(2)));

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16-byte HBM -> LDS copy per lane (global_load_lds_dwordx4): lane i's bytes
// land at dst + 16 i; dst must be wave-uniform. The builtin exists only for
// the device pass (clang drops the kernel's host stub if the host pass sees it).
__device__ __forceinline__ void copy16_to_lds(const void* src, lds_ptr_t dst) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
#endif
}

// True when wasm_h2f of each of the four fp16 values packed in w is the
// hardware widening: every value is zero or normal (no subnormal, inf or
// NaN). Per half h = bits & 0x7fff, with packed 16-bit arithmetic:
// (h - 1) mod 2^16 >= 0x3ff excludes the subnormals (zero wraps to 0xffff)
// and h < 0x7c00 excludes inf and NaN.
__device__ __forceinline__ bool h4_normal(u2_t w) {
  const us2_t one = {1, 1};
  const us2_t hx = __builtin_bit_cast(us2_t, w.x & 0x7fff7fffu), hy = __builtin_bit_cast(us2_t, w.y & 0x7fff7fffu);
  const us2_t lo = __builtin_elementwise_min(hx - one, hy - one);
  const us2_t hi = __builtin_elementwise_max(hx, hy);
  return (lo.x >= 0x3ff) & (lo.y >= 0x3ff) & (hi.x < 0x7c00) & (hi.y < 0x7c00);
}

__device__ __noinline__ f4_t h4_widen_exact(u2_t w) {
  return f4_t{wasm_h2f((uint16_t)(w.x & 0xFFFFu)), wasm_h2f((uint16_t)(w.x >> 16)),
              wasm_h2f((uint16_t)(w.y & 0xFFFFu)), wasm_h2f((uint16_t)(w.y >> 16))};
}

// wasm_h2f of four packed fp16 values: the hardware widening when all are
// zero or normal, the exact software path (not inlined) otherwise.
__device__ __forceinline__ void h4_widen(u2_t w, float v[4]) {
  if (h4_normal(w)) {
    v[0] = hw_h2f((uint16_t)(w.x & 0xFFFFu));
    v[1] = hw_h2f((uint16_t)(w.x >> 16));
    v[2] = hw_h2f((uint16_t)(w.y & 0xFFFFu));
    v[3] = hw_h2f((uint16_t)(w.y >> 16));
  } else {
    const f4_t e = h4_widen_exact(w);
    v[0] = e[0];
    v[1] = e[1];
    v[2] = e[2];
    v[3] = e[3];
  }
}

// f32 -> exact (hi, lo) fp16 pair: hi = fp16(v), lo = fp16(v - hi); hi + lo
// carries 22 significant bits of v (the form SPLIT GEMM inputs take).
__device__ __forceinline__ void split_hilo(float v, uint16_t& hi, uint16_t& lo) {
  v = f32_fence(v);
  const _Float16 h = (_Float16)v;
  const _Float16 l = (_Float16)(v - (float)h);
  hi = __builtin_bit_cast(uint16_t, h);
  lo = __builtin_bit_cast(uint16_t, l);
}

// expApproxNonPositiveF32x4 (zig/wasm_exports.zig:812-838), one lane.
// Accuracy ~2.8e-4 relative; reproduced, not replaced, so GPU softmax and
// SwiGLU track the reference's values.
__device__ __forceinline__ float exp_approx(float x) {
  const float LOG2_E = 1.44269504088896340736f;
  float clamped = fmaxf(x, -88.0f);
  float y = clamped * LOG2_E;
  float fl = floorf(y);
  int32_t iv = (int32_t)fl;
  float frac = y - (float)iv;
  float poly = fmaf(0.001333355f, frac, 0.009679494f);
  poly = fmaf(poly, frac, 0.055053319f);
  poly = fmaf(poly, frac, 0.240226522f);
  poly = fmaf(poly, frac, 0.693154774f);
  poly = fmaf(poly, frac, 1.000000012f);
  float scale = __uint_as_float((uint32_t)(iv + 127) << 23);
  return poly * scale;
}

// exp_approx with the final scaling done by ldexp. The two give the same
// value unless floor(x log2 e) = -127 (x < -87.3), where exp_approx returns
// 0 and this a value below 2^-126 (tests/test_gpu_kernels.py checks every
// other f32 x <= 0 exhaustively). Callers use it where such a difference
// cannot reach their output (see each call site).
__device__ __forceinline__ float exp_approx_fast(float x) {
  const float LOG2_E = 1.44269504088896340736f;
  const float y = fmaxf(x, -88.0f) * LOG2_E;
  const float fl = floorf(y);
  const float frac = y - fl;  // fl is an integer of magnitude <= 127: y - (float)(int)fl
  float poly = fmaf(0.001333355f, frac, 0.009679494f);
  poly = fmaf(poly, frac, 0.055053319f);
  poly = fmaf(poly, frac, 0.240226522f);
  poly = fmaf(poly, frac, 0.693154774f);
  poly = fmaf(poly, frac, 1.000000012f);
  return __builtin_amdgcn_ldexpf(poly, (int)fl);
}

// e / (1 + e) for e in [0, 1], correctly rounded: hardware reciprocal of
// b = 1 + e refined by one Newton-Raphson step, then one remainder
// correction of the quotient (Markstein 1990; Cornea-Hasegan, Golliver and
// Markstein 1999). tests/test_gpu_kernels.py compares it with IEEE division
// for every f32 e in [0, 1].
__device__ __forceinline__ float div_one_plus(float e) {
  const float b = 1.0f + e;
  float r = __builtin_amdgcn_rcpf(b);
  r = fmaf(fmaf(-b, r, 1.0f), r, r);
  const float q = e * r;
  return fmaf(fmaf(-b, q, e), r, q);
}

// sigmoidF32x4 (zig/wasm_exports.zig:843-853), one lane:
// neg_abs = min(x, 0) - max(x, 0) (= -|x|), e = expApprox(neg_abs),
// sig_neg = e / (1 + e), x >= 0 ? 1 - sig_neg : sig_neg.
__device__ __forceinline__ float sigmoid_approx(float x) {
  const float sig_neg = div_one_plus(exp_approx(-fabsf(x)));
  return x >= 0.0f ? 1.0f - sig_neg : sig_neg;
}
// The same with exp_approx_fast: e differs only for |x| > 87.3, where
// e < 2^-126, 1 - sig_neg = 1 exactly and sig_neg < 2^-126 either way.
__device__ __forceinline__ float sigmoid_approx_fast(float x) {
  const float sig_neg = div_one_plus(exp_approx_fast(-fabsf(x)));
  return x >= 0.0f ? 1.0f - sig_neg : sig_neg;
}

// SwiGLU with clamp (zig/wasm_exports.zig:855-903 vector path).
__device__ __forceinline__ float swiglu_clamp(float gate_raw, float up_raw) {
  const float gate = fminf(gate_raw, 7.0f);
  const float up = fmaxf(fminf(up_raw, 7.0f), -7.0f);
  return (up + 1.0f) * (gate * sigmoid_approx(gate * 1.702f));
}
// The same for outputs stored as fp16 or hi/lo fp16: where the fast
// sigmoid differs (gate < -51.3) the result is below 2^-120 in magnitude and
// both round to a zero fp16 (hi and lo).
__device__ __forceinline__ float swiglu_clamp_fast(float gate_raw, float up_raw) {
  const float gate = fminf(gate_raw, 7.0f);
  const float up = fmaxf(fminf(up_raw, 7.0f), -7.0f);
  return (up + 1.0f) * (gate * sigmoid_approx_fast(gate * 1.702f));
}

// SwiGLU with the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32; each
// within about 1 ulp), for the fp16 forward, which follows the GPU paths'
// numerics (src/native/shaders/swiglu_clamp.wgsl:10-25 uses the WGSL exp).
// sigma(x) = 1 / (1 + exp(-x)) needs no branch here: for very negative x the
// hardware exp2 returns +inf and its reciprocal 0. alpha * log2(e) is folded
// into one constant. The result differs from swiglu_clamp by a few f32 ulps,
// which changes an fp16-rounded output in about one case in a thousand, by
// one fp16 ulp (plus the reference polynomial's own error, ~1e-4 relative,
// which the GPU paths do not have).
// SETTLED: the operands are MFMA results that have passed through
// mfma_settled (below), so min(gate, 7) can be one v_min_f32 in inline
// assembly (fminf first quiets its operand, one more instruction per value,
// which MFMA results never need; a quiet NaN yields 7 either way). Otherwise
// fminf: the matrix cores write a result several cycles after the MFMA
// issues, and the compiler inserts those wait states only before the
// instructions it can see.
template <bool SETTLED = false>
__device__ __forceinline__ float swiglu_clamp_hw(float gate_raw, float up_raw) {
  float gate;
  if constexpr (SETTLED) asm("v_min_f32 %0, 0x40e00000, %1" : "=v"(gate) : "v"(gate_raw));
  else gate = fminf(gate_raw, 7.0f);
  const float up = __builtin_amdgcn_fmed3f(up_raw, -7.0f, 7.0f);
  constexpr float NEG_ALPHA_LOG2E = -1.702f * 1.44269504088896340736f;
  const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gate * NEG_ALPHA_LOG2E));
  return (up + 1.0f) * (gate * sig);
}

// Eight wait states after the MFMAs that wrote the n accumulators (the
// operands order it after them): what a dependent read of an MFMA result
// needs on gfx950 from an instruction the compiler does not see.
template <int N>
__device__ __forceinline__ void mfma_settled(f4_t (&a)[N]) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8, "1, 2, 4 or 8 accumulators");
  if constexpr (N == 1) asm volatile("s_nop 7" : "+v"(a[0]));
  if constexpr (N == 2) asm volatile("s_nop 7" : "+v"(a[0]), "+v"(a[1]));
  if constexpr (N == 4) asm volatile("s_nop 7" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]));
  if constexpr (N == 8)
    asm volatile("s_nop 7"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7]));
}

// v_mfma_f32_16x16x32_f16 (gfx950). Operand layout (lane l, i = l / 16):
//   a: A[m = l%16][k = 8i .. 8i+7]     (16 x 32, row-major fragment)
//   b: B[k = 8i .. 8i+7][n = l%16]     (32 x 16)
//   c/d: D[m = 4i + r][n = l%16], r = 0..3
// The layout is checked on the GPU by tests/test_gpu_kernels.py
// (probe_mfma_f16) against a host matrix product.
__device__ __forceinline__ f4_t mfma16x16x32(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Wave-wide reductions over 64 lanes.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace pf
