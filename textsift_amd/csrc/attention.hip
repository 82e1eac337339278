// attention.hip — banded (sliding-window) bidirectional GQA attention with
// per-head sinks for gfx950.
//
// Reference semantics: bandedAttentionBody, packages/textsift/src/zig/
// wasm_exports.zig:1286-1378. For query t of head h (kv head h / (Hq/Hkv)):
// keys ws = max(0, t-W) .. we = min(T, t+W+1); scores = q.k (times `scale`);
// m = max(sink, valid scores); e_i = expApprox(s_i - m) for the reference's
// 4-lane vector part and libm exp for its scalar tail; p_i = e_i / sum(e, sink);
// out = fp16(sum_i p_i v_i). Masked keys score -inf.
//
// Mapping to CDNA4 (one workgroup = 4 waves = 64 query tokens of one
// sequence and one KV head, all Hq/Hkv query heads of that group):
//  * The workgroup stages its union of keys (64 + 2W rows) once in LDS:
//    K row-major, V transposed (V^T[dim][key]); every query head of the
//    group reuses them.
//  * S^T = K . Q^T on v_mfma_f32_16x16x32_f16 leaves each lane holding 4
//    consecutive keys of one query; two such 16-key tiles are exactly the
//    B-operand fragment of the P.V MFMA (O^T = V^T . P^T), so P never
//    leaves registers.
//  * Because the whole band (<= 2W+16 keys per 16-query wave tile) fits in
//    registers, the softmax is the reference's two-pass one (global max
//    first, then exp), not an online rescaling: probabilities match the
//    reference's values, not just its mathematics.
//  * p is normalised before P.V (as the reference does) and enters the
//    MFMA as an fp16 hi + lo pair, so P.V carries ~22 significant bits.
#include "common.h"
#include "epilogue.h"
#include "pfhip_internal.h"

namespace pf {

namespace {

// The softmax uses exp_approx_fast where the reference uses expApprox. They
// differ only when floor(x log2 e) = -127 (x < -87.3): such a term is below
// 2^-126 of the row maximum's (which is 1), so it leaves the f32 row sum
// unchanged and its probability rounds to fp16 zero in both hi and lo: the
// attention output is identical.
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  return __builtin_amdgcn_readfirstlane(v);
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return __builtin_amdgcn_readfirstlane(v);
}

// LDS geometry of a workgroup of NW waves x 16 queries with NCH 32-key
// chunks per wave: ROWS staged keys (every wave's chunks, rounded up to 32),
// K row-major [ROWS][LDK], V transposed [HD][LDV]. LDK = HD + 8 halves
// (36 dwords for HD = 64: the 16-byte K-fragment reads of 8 consecutive rows
// hit distinct banks); LDV = ROWS + 4 halves (2 mod 4 dwords: the 8-byte
// V^T-fragment reads of 16 consecutive rows hit distinct banks).
template <int HD, int NCH, int NW>
struct AttnGeom {
  static constexpr int ROWS = (16 * (NW - 1) + 32 * NCH + 31) / 32 * 32;
  static constexpr int LDK = HD + 8;
  static constexpr int LDV = ROWS + 4;
  static constexpr size_t LDS = (size_t)(ROWS * LDK + HD * LDV) * 2;
  static_assert(LDV % 8 == 4, "V^T row stride must be 2 mod 4 dwords");
};

// Stages the workgroup's keys kbase .. kbase + ROWS - 1 of kv head g into
// Ks / Vt (layout of AttnGeom); V rows outside [0, T) are zero, K rows
// outside [0, T) are zero with ZERO_K and otherwise not written (their
// scores are masked before any use). Every load is issued before any is waited for: K goes HBM ->
// LDS directly (global_load_lds, 16-byte units; a K row of LDK halves is
// LDK / 8 units, the last of which is padding and copies the row's first
// unit), V is loaded into registers and written transposed. Ends with the
// workgroup barrier.
template <int HD, int ROWS, int LDK, int LDV, int NT, bool ZERO_K = true>
__device__ __forceinline__ void stage_kv(const AttnArgs& a, _Float16* Ks, _Float16* Vt, size_t seq0, int g, int kbase,
                                         int tid) {
  static_assert(ROWS % 32 == 0, "V^T staging: whole groups of 8 x 4 keys");
  static_assert(LDK % 8 == 0 && LDK > HD, "K rows of whole 16-byte units");
  const int T = a.T;
  const int wave = tid >> 6;
  constexpr int UPR = LDK / 8;  // 16-byte units per staged K row
  constexpr int NK = ROWS * UPR, IK = (NK + NT - 1) / NT;
#pragma unroll
  for (int it = 0; it < IK; ++it) {
    const int u = it * NT + tid;
    const int r = u / UPR, c = u % UPR;
    const int key = kbase + r;
    if (u < NK && key >= 0 && key < T)  // rows outside [0, T) are cleared below
      copy16_to_lds(a.k + (seq0 + key) * a.k_stride + g * HD + (c < HD / 8 ? c : 0) * 8,
                    (lds_ptr_t)(Ks + (size_t)(it * NT + wave * 64) * 8));
  }
  // 4 keys x 8 dims per thread; 8 consecutive lanes take 32 consecutive keys
  // of the same 8 dims, so each V^T row write of 16 lanes covers distinct banks
  constexpr int NV = (ROWS / 4) * (HD / 8), IV = (NV + NT - 1) / NT;
  u4_t vv[IV][4];
#pragma unroll
  for (int it = 0; it < IV; ++it) {
    const int i = min(it * NT + tid, NV - 1);
    const int c = (i >> 3) % (HD / 8), r4 = ((i & 7) + 8 * ((i >> 3) / (HD / 8))) * 4;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int key = kbase + r4 + u;
      const u4_t v = *reinterpret_cast<const u4_t*>(a.v + (seq0 + min(max(key, 0), T - 1)) * a.v_stride + g * HD + c * 8);
      vv[it][u] = key >= 0 && key < T ? v : u4_t{0u, 0u, 0u, 0u};
    }
  }
#pragma unroll
  for (int it = 0; it < IV; ++it) {
    const int i = it * NT + tid;
    if (i < NV) {
      const int c = (i >> 3) % (HD / 8), r4 = ((i & 7) + 8 * ((i >> 3) / (HD / 8))) * 4;
      h8_t vh[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) vh[u] = __builtin_bit_cast(h8_t, vv[it][u]);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        *reinterpret_cast<h4_t*>(&Vt[(c * 8 + j) * LDV + r4]) = h4_t{vh[0][j], vh[1][j], vh[2][j], vh[3][j]};
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the K copies
  __syncthreads();
  if (ZERO_K && (kbase < 0 || kbase + ROWS > T)) {  // at a sequence end: clear the K rows outside [0, T)
    for (int u = tid; u < NK; u += NT) {
      const int key = kbase + u / UPR;
      if (key < 0 || key >= T) *reinterpret_cast<u4_t*>(Ks + (size_t)u * 8) = u4_t{0u, 0u, 0u, 0u};
    }
    __syncthreads();
  }
}

// The WASM path's numerics (split): polynomial expApprox for the
// reference's 4-lane part, libm exp for its scalar tail, p normalised before
// P.V. NW waves x 16 queries per workgroup; NCH 32-key chunks per 16-query
// tile.
template <int HD, int NCH, int NW>
__global__ __launch_bounds__(64 * NW) void k_banded_attention(AttnArgs a) {
  using GE = AttnGeom<HD, NCH, NW>;
  constexpr int QB = 16 * NW;                // query tokens per workgroup
  constexpr int ROWS = GE::ROWS, LDK = GE::LDK, LDV = GE::LDV;
  constexpr int NDH = HD / 32;               // MFMA K-steps over head_dim for Q.K
  constexpr int NDT = HD / 16;               // 16-row dim tiles of O^T
  extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
  _Float16* Ks = smem;                       // [ROWS][LDK]
  _Float16* Vt = smem + ROWS * LDK;          // [HD][LDV]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int t0 = blockIdx.x * QB;
  const int g = blockIdx.y / a.head_groups;  // kv head
  const int hgrp = blockIdx.y % a.head_groups;  // which of its query heads this workgroup takes
  const int bseq = blockIdx.z;
  const int T = a.T, W = a.window;
  const size_t seq0 = (size_t)bseq * T;
  const int kbase = t0 - W;                  // key index of staged row 0

  stage_kv<HD, ROWS, LDK, LDV, 64 * NW>(a, Ks, Vt, seq0, g, kbase, tid);

  const int tq0 = t0 + 16 * wave;            // this wave's first query
  const int tq = tq0 + l16;                  // this lane's query
  const int rb = 16 * wave;                  // staged row of key tq0 - W
  const int kw = tq0 - W;                    // key at chunk offset 0 of this wave
  const bool q_ok = tq < T;
  const int ws = max(0, tq - W), we = min(T, tq + W + 1);
  const int n_keys = we - ws;
  const int total = n_keys + 1;
  const int vec_end = total - (total & 3);   // reference's 4-lane part vs scalar tail
  // window [lo, hi) and scalar tail [tail, hi) as chunk offsets
  const int lo0 = ws - kw, hi0 = we - kw, tail0 = ws + vec_end - kw;
  // wave-uniform chunk classes (lanes past T do not constrain them)
  const int full_lo = wave_max_i(q_ok ? lo0 : 0);
  const int full_hi = wave_min_i(q_ok ? hi0 : 1 << 20);
  const int tail_lo = wave_min_i(q_ok ? tail0 : 1 << 20);
  const int any_hi = wave_max_i(q_ok ? hi0 : 0);
  const bool masked = a.mask != nullptr;
  const int G = a.Hq / a.Hkv;
  const float sscale = a.scale;

  // this workgroup's query heads: an even split of the group's G heads
  for (int hh = hgrp * G / a.head_groups; hh < (hgrp + 1) * G / a.head_groups; ++hh) {
    const int hq = g * G + hh;
    // Opaque per-head copies of the window bounds: comparisons against them
    // are then recomputed per head instead of being hoisted out of the loop
    // as dozens of live lane masks (which spill).
    int lo = lo0, hi = hi0, tail = tail0;
    asm volatile("" : "+v"(lo), "+v"(hi), "+v"(tail));
    // Q fragment (B operand): Q[tq][32 dh + 8 lg .. +8]
    h8_t qf[NDH];
#pragma unroll
    for (int dh = 0; dh < NDH; ++dh) {
      u4_t v = {0u, 0u, 0u, 0u};
      if (q_ok) v = *reinterpret_cast<const u4_t*>(a.q + (seq0 + tq) * a.q_stride + hq * HD + 32 * dh + 8 * lg);
      qf[dh] = __builtin_bit_cast(h8_t, v);
    }
    const float sink = a.sinks ? a.sinks[hq] : -INFINITY;

    // ---- pass 1: scores for the whole band, kept in registers. Slots
    // outside the query's window hold NaN; masked keys hold -inf.
    float s[NCH][2][4];
    float m = sink;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      f4_t acc[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        acc[kt] = f4_t{0.f, 0.f, 0.f, 0.f};
        const int row = rb + 32 * c + 16 * kt + l16;
#pragma unroll
        for (int dh = 0; dh < NDH; ++dh) {
          const h8_t kf = *reinterpret_cast<const h8_t*>(&Ks[row * LDK + 32 * dh + 8 * lg]);
          acc[kt] = mfma16x16x32(kf, qf[dh], acc[kt]);
        }
      }
      if (!masked && 32 * c >= full_lo && 32 * c + 32 <= full_hi) {  // every slot in every window
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float sv = acc[kt][r] * sscale;
            s[c][kt][r] = sv;
            m = fmaxf(m, sv);
          }
      } else {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int off = 32 * c + 16 * kt + 4 * lg + r;
            const bool inwin = (off >= lo) & (off < hi);
            bool valid = inwin;
            if (masked) valid = valid && a.mask[seq0 + kw + off] != 0;
            const float sv = valid ? acc[kt][r] * sscale : -INFINITY;
            s[c][kt][r] = inwin ? sv : NAN;
            m = valid ? fmaxf(m, sv) : m;
          }
      }
      // keep the scheduler from hoisting every chunk's LDS loads (spills)
      __builtin_amdgcn_sched_barrier(0);
    }
    // lanes l, l^16, l^32, l^48 hold the same query
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));

    // ---- pass 2: exp (polynomial in the reference's vector part, libm in
    // its scalar tail) and the row sum
    float l = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const bool plain = !masked && 32 * c >= full_lo && 32 * c + 32 <= full_hi &&
                         !(32 * c + 32 > tail_lo && 32 * c < any_hi);
      if (plain) {  // wave-uniform: every slot in every window, no tail key
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float e = exp_approx_fast(s[c][kt][r] - m);
            s[c][kt][r] = e;
            l += e;
          }
      } else {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float sv = s[c][kt][r];
            const float x = sv - m;
            const int off = 32 * c + 16 * kt + 4 * lg + r;
            float e = off >= tail ? expf(x) : exp_approx_fast(x);
            e = (sv != sv) ? 0.0f : e;
            s[c][kt][r] = e;
            l += e;
          }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    l += n_keys < vec_end ? exp_approx_fast(sink - m) : expf(sink - m);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;

    // ---- pass 3: O^T = V^T . P^T with P normalised, as fp16 hi + lo
    f4_t o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      h8_t ph, pl;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv = f32_fence(s[c][kt][r] * inv);  // split the f32 probability
          const _Float16 hi16 = (_Float16)pv;
          ph[4 * kt + r] = hi16;
          pl[4 * kt + r] = (_Float16)(pv - (float)hi16);
        }
      const int row = rb + 32 * c + 4 * lg;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const _Float16* vr = &Vt[(16 * dt + l16) * LDV + row];
        const h4_t v0 = *reinterpret_cast<const h4_t*>(vr);
        const h4_t v1 = *reinterpret_cast<const h4_t*>(vr + 16);
        const h8_t vf = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        o[dt] = mfma16x16x32(vf, ph, o[dt]);
        o[dt] = mfma16x16x32(vf, pl, o[dt]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // lane holds out[tq][hq*HD + 16 dt + 4 lg + r]
    if (q_ok) {
      uint16_t* orow = a.out + (seq0 + tq) * a.out_stride + hq * HD;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const float ov[4] = {o[dt][0], o[dt][1], o[dt][2], o[dt][3]};
        *reinterpret_cast<u2_t*>(orow + 16 * dt + 4 * lg) = to_f16x4(ov);
      }
    }
  }
}


// The reference's GPU-path numerics (fp16): the softmax exponentials use the
// hardware exp2 (v_exp_f32, about 1 ulp) on scores in units of log2(e), as
// the GPU shader uses the WGSL exp (native/shaders/banded_attention.wgsl:
// 100-113), and the output is stored with the hardware fp16 conversion.
// After the max pass, one pass per 32-key chunk computes e = 2^(s - m),
// rounds it to an fp16 weight and feeds it straight into P.V and the row sum,
// so the exponentials of one chunk overlap the MFMAs of the previous one; the
// normalisation by the row sum is applied to the f32 output accumulators
// (sum_i (p_i / l) v_i = (sum_i p_i v_i) / l up to f32 rounding). The shader
// keeps f32 weights; the fp16 weight is this path's one extra rounding
// (output error ~3e-4 relative against the shader's f32 weights). Requires
// scale > 0 (the row maximum is taken over the unscaled scores).
// max(a, b, c) in one v_max3_f32. Written as assembly: the compiler's
// fmaxf quiets each operand first (signalling NaNs), which MFMA results and
// -inf never are. Its operands are MFMA results, and the compiler counts the
// wait states before a read of those only for instructions it can see: the
// scores pass through mfma_settled first.
__device__ __forceinline__ float max3_f32(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}


// MASKED: a key mask is given (a compile-time choice, so the unmasked
// kernel carries no per-slot mask code)
template <int HD, int NCH, int NW, bool MASKED>
__global__ __launch_bounds__(64 * NW) void k_banded_attention_hw(AttnArgs a) {
  using GE = AttnGeom<HD, NCH, NW>;
  constexpr int QB = 16 * NW;                // query tokens per workgroup
  constexpr int ROWS = GE::ROWS, LDK = GE::LDK, LDV = GE::LDV;
  constexpr int NDH = HD / 32;               // MFMA K-steps over head_dim for Q.K
  constexpr int NDT = HD / 16;               // 16-row dim tiles of O^T
  extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
  _Float16* Ks = smem;                       // [ROWS][LDK]
  _Float16* Vt = smem + ROWS * LDK;          // [HD][LDV]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int t0 = blockIdx.x * QB;
  const int g = blockIdx.y / a.head_groups;  // kv head
  const int hgrp = blockIdx.y % a.head_groups;  // which of its query heads this workgroup takes
  const int bseq = blockIdx.z;
  const int T = a.T, W = a.window;
  const size_t seq0 = (size_t)bseq * T;
  const int kbase = t0 - W;                  // key index of staged row 0

  // (K rows outside the sequence stay unwritten: every score of one is
  // replaced by -inf before the maximum and the exponentials)
  stage_kv<HD, ROWS, LDK, LDV, 64 * NW, false>(a, Ks, Vt, seq0, g, kbase, tid);

  const int tq0 = t0 + 16 * wave;            // this wave's first query
  const int tq = tq0 + l16;                  // this lane's query
  const int rb = 16 * wave;                  // staged row of key tq0 - W
  const int kw = tq0 - W;                    // key at chunk offset 0 of this wave
  const bool q_ok = tq < T;
  const int ws = max(0, tq - W), we = min(T, tq + W + 1);
  const int lo0 = ws - kw, hi0 = we - kw;    // the window [lo, hi) as chunk offsets
  // wave-uniform: chunks wholly inside every lane's window (lanes past T do not constrain them)
  const int full_lo = wave_max_i(q_ok ? lo0 : 0);
  const int full_hi = wave_min_i(q_ok ? hi0 : 1 << 20);
  // chunks outside every lane's window (near the sequence ends) are skipped
  const int any_lo = wave_min_i(q_ok ? lo0 : 1 << 20);
  const int any_hi = wave_max_i(q_ok ? hi0 : -1);
  auto empty = [&](int c) { return 32 * c + 32 <= any_lo || 32 * c >= any_hi; };
  constexpr bool masked = MASKED;
  const int G = a.Hq / a.Hkv;
  constexpr float LOG2_E = 1.44269504088896340736f;
  const float sscale = a.scale * LOG2_E;     // scores in the exponent's units

  // this workgroup's query heads: an even split of the group's G heads. The
  // next head's Q fragments are loaded while this head is processed.
  const int h_end = (hgrp + 1) * G / a.head_groups;
  auto load_q = [&](int hq, h8_t (&dst)[NDH]) {
#pragma unroll
    for (int dh = 0; dh < NDH; ++dh) {
      const u4_t v = *reinterpret_cast<const u4_t*>(a.q + (seq0 + min(tq, T - 1)) * a.q_stride + hq * HD + 32 * dh +
                                                    8 * lg);
      dst[dh] = __builtin_bit_cast(h8_t, q_ok ? v : u4_t{0u, 0u, 0u, 0u});
    }
  };
  // (raw values: scaled where used, so the load is not waited for at once)
  auto load_sink = [&](int hq) { return a.sinks ? a.sinks[hq] : -INFINITY; };
  h8_t qf[NDH];
  float sink = load_sink(g * G + hgrp * G / a.head_groups);
  load_q(g * G + hgrp * G / a.head_groups, qf);
  for (int hh = hgrp * G / a.head_groups; hh < h_end; ++hh) {
    const int hq = g * G + hh;
    // opaque per-head copies of the window bounds (see k_banded_attention)
    int lo = lo0, hi = hi0;
    asm volatile("" : "+v"(lo), "+v"(hi));
    const int hn = hh + 1 < h_end ? hq + 1 : hq;
    const float sink_n = load_sink(hn);  // issued before the Q loads: waiting for it leaves them in flight
    h8_t qn[NDH];
    load_q(hn, qn);

    // ---- pass 1: unscaled scores for the whole band, kept in registers;
    // slots outside the query's window and masked keys hold -inf. The K
    // fragments of chunk c + 1 are read while chunk c is processed. The
    // MFMAs write the score registers themselves and edge chunks are masked
    // in place (no copies between register sets); the running maximum takes
    // three values per instruction.
    f4_t s[NCH][2];
    float mr = -INFINITY;
    // K fragments double-buffered by chunk parity (compile-time indices once
    // the chunk loop is unrolled: no register copies between chunks)
    h8_t kb[2][2][NDH];
    auto load_k = [&](int c, h8_t (&dst)[2][NDH]) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int dh = 0; dh < NDH; ++dh)
          dst[kt][dh] = *reinterpret_cast<const h8_t*>(&Ks[(rb + 32 * c + 16 * kt + l16) * LDK + 32 * dh + 8 * lg]);
    };
    load_k(0, kb[0]);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c + 1 < NCH) load_k(c + 1, kb[(c + 1) & 1]);
      const h8_t (&kf)[2][NDH] = kb[c & 1];
      if (empty(c)) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) s[c][kt] = f4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      } else {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) s[c][kt] = mfma16x16x32(kf[kt][0], qf[0], f4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int dh = 1; dh < NDH; ++dh)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) s[c][kt] = mfma16x16x32(kf[kt][dh], qf[dh], s[c][kt]);
        if (masked || 32 * c < full_lo || 32 * c + 32 > full_hi) {
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int off = 32 * c + 16 * kt + 4 * lg + r;
              bool valid = (off >= lo) & (off < hi);
              if constexpr (MASKED) valid = valid && a.mask[seq0 + kw + off] != 0;
              s[c][kt][r] = valid ? s[c][kt][r] : -INFINITY;
            }
        }
        mfma_settled(s[c]);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          mr = max3_f32(mr, s[c][kt][0], s[c][kt][1]);
          mr = max3_f32(mr, s[c][kt][2], s[c][kt][3]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // lanes l, l^16, l^32, l^48 hold the same query
    mr = fmaxf(mr, __shfl_xor(mr, 16, 64));
    mr = fmaxf(mr, __shfl_xor(mr, 32, 64));
    // max over the scaled scores (scaling by sscale > 0 keeps the order) and the sink;
    // -inf only without a sink and with no valid key (every e is then 0)
    const float sink2 = sink * LOG2_E;
    float m = fmaxf(mr * sscale, sink2);
    m = m == -INFINITY ? 0.0f : m;
    const float nm = -m;

    // ---- pass 2: e = 2^(s sscale - m), the row sum, and O^T += V^T . P^T
    // with P = e rounded once to fp16 (toward zero: one conversion per two
    // values). The row sum runs on the matrix cores too: an all-ones A
    // operand gives every output row sum_k P_k for the lane's query, so the
    // normalisation divides by the sum of exactly the weights used and the
    // rounding only perturbs the weights relative to each other (by under
    // 2^-10). The V^T fragments of chunk c + 1 are read while chunk c is
    // processed.
    const h8_t ones = {1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16};
    f4_t lsum = f4_t{0.f, 0.f, 0.f, 0.f};
    f4_t o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
    h8_t vb[2][NDT];  // V^T fragments double-buffered by chunk parity
    auto load_v = [&](int c, h8_t (&dst)[NDT]) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const _Float16* vr = &Vt[(16 * dt + l16) * LDV + rb + 32 * c + 4 * lg];
        const h4_t v0 = *reinterpret_cast<const h4_t*>(vr);
        const h4_t v1 = *reinterpret_cast<const h4_t*>(vr + 16);
        dst[dt] = h8_t{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      }
    };
    // e of chunk c as the fp16 B operand
    auto probs = [&](int c, h8_t& pf) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          const float e0 = __builtin_amdgcn_exp2f(fmaf(s[c][kt][r], sscale, nm));
          const float e1 = __builtin_amdgcn_exp2f(fmaf(s[c][kt][r + 1], sscale, nm));
          const h2_t ph = __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_pkrtz(e0, e1));
          pf[4 * kt + r] = ph[0];
          pf[4 * kt + r + 1] = ph[1];
        }
    };
    auto pv = [&](const h8_t (&vf)[NDT], const h8_t& pf) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] = mfma16x16x32(vf[dt], pf, o[dt]);
      lsum = mfma16x16x32(ones, pf, lsum);
    };
    // pass 2 (exponentials and P.V) at raised wave priority: the waves in it
    // issue ahead of those in the max pass (-1.7 us)
    __builtin_amdgcn_s_setprio(1);
    load_v(0, vb[0]);
    if (!empty(0) && !empty(NCH - 1)) {
      // every chunk has keys (all but the sequence ends): one branch-free
      // block in which chunk c + 1's exponentials are computed before chunk
      // c's MFMAs are issued, so the compiler can interleave the two
      h8_t pb[2];  // by parity
      probs(0, pb[0]);
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if (c + 1 < NCH) {
          load_v(c + 1, vb[(c + 1) & 1]);
          probs(c + 1, pb[(c + 1) & 1]);
        }
        pv(vb[c & 1], pb[c & 1]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if (c + 1 < NCH) load_v(c + 1, vb[(c + 1) & 1]);
        if (!empty(c)) {
          h8_t pf;
          probs(c, pf);
          pv(vb[c & 1], pf);
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
    const float l = lsum[0] + __builtin_amdgcn_exp2f(sink2 - m);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    // lane holds out[tq][hq*HD + 16 dt + 4 lg + r]
    if (q_ok) {
      uint16_t* orow = a.out + (seq0 + tq) * a.out_stride + hq * HD;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const float ov[4] = {o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv};
        *reinterpret_cast<u2_t*>(orow + 16 * dt + 4 * lg) = to_f16x4_native(ov);
      }
    }
#pragma unroll
    for (int dh = 0; dh < NDH; ++dh) qf[dh] = qn[dh];
    sink = sink_n;
  }
}

template <typename Kern>
void launch_kernel(pfhip_backend* b, const AttnArgs& a, Kern* kern, size_t lds, int qb, int nt) {
  allow_lds(reinterpret_cast<const void*>(kern), lds);
  // few workgroups (short inputs): the query heads of a KV head are split
  // over several workgroups (the fewest that give every CU one), so they run
  // in parallel; each still stages its K/V rows once for all its heads
  AttnArgs g = a;
  const long wgs = (long)((a.T + qb - 1) / qb) * a.Hkv * a.B;
  const int G = a.Hq / a.Hkv;
  g.head_groups = (int)std::min<long>(G, (b->num_cus + wgs - 1) / wgs);
  dim3 grid((a.T + qb - 1) / qb, a.Hkv * g.head_groups, a.B);
  ProfScope ps(b, "banded_attention");
  hipLaunchKernelGGL(kern, grid, dim3(nt), lds, b->stream, g);
  PF_HIP(hipGetLastError());
}

template <int HD, int NCH, int NW>
void launch_attn(pfhip_backend* b, const AttnArgs& a) {
  constexpr size_t LDS = AttnGeom<HD, NCH, NW>::LDS;
  static_assert(LDS <= 160 * 1024, "attention tile exceeds the LDS");
  if (a.hw_exp) {
    if (a.mask) launch_kernel(b, a, &k_banded_attention_hw<HD, NCH, NW, true>, LDS, 16 * NW, 64 * NW);
    else launch_kernel(b, a, &k_banded_attention_hw<HD, NCH, NW, false>, LDS, 16 * NW, 64 * NW);
  } else {
    launch_kernel(b, a, &k_banded_attention<HD, NCH, NW>, LDS, 16 * NW, 64 * NW);
  }
}

template <int HD>
void pick_nch(pfhip_backend* b, const AttnArgs& a) {
  const int need = (16 + 2 * a.window + 31) / 32;  // 32-key chunks per 16-query tile
  if (need <= 1) return launch_attn<HD, 1, 4>(b, a);
  if (need <= 2) return launch_attn<HD, 2, 4>(b, a);
  if (need <= 3) return launch_attn<HD, 3, 4>(b, a);
  if (need <= 5) return launch_attn<HD, 5, 8>(b, a);
  return launch_attn<HD, 9, 8>(b, a);
}

}  // namespace

void banded_attention(pfhip_backend* b, const AttnArgs& a) {
  PF_CHECK(a.head_dim == 64 || a.head_dim == 32, "banded_attention: head_dim must be 32 or 64");
  PF_CHECK(a.Hkv > 0 && a.Hq % a.Hkv == 0, "banded_attention: Hq must be a multiple of Hkv");
  // 16 + 2W keys per 16-query tile must fit nine 32-key chunks (LDS: 110 KB)
  PF_CHECK(a.window >= 0 && a.window <= 128, "banded_attention: window must be in [0, 128]");
  PF_CHECK(a.q && a.k && a.v && a.out, "banded_attention: null operand");
  PF_CHECK(!a.hw_exp || a.scale > 0.0f, "banded_attention: the hardware-exp softmax needs scale > 0");
  PF_CHECK(a.q_stride % 8 == 0 && a.k_stride % 8 == 0 && a.v_stride % 8 == 0 && a.out_stride % 4 == 0,
           "banded_attention: row strides must allow 16-byte loads");
  PF_CHECK(((uintptr_t)a.q & 15) == 0 && ((uintptr_t)a.k & 15) == 0 && ((uintptr_t)a.v & 15) == 0 &&
               ((uintptr_t)a.out & 7) == 0,
           "banded_attention: operands must be 16-byte aligned");
  if (a.B <= 0 || a.T <= 0) return;
  // A sequence no longer than the window attends to all of itself: any window
  // of at least T - 1 gives every query the same keys. The GPU-shader kernel
  // then runs with the smallest such window that differs from the given one
  // by a multiple of 32: its 32-key chunks hold the same keys in the same
  // order (so the results are the same bits), and the tile stages and skips
  // fewer of them (T = 7: 160 instead of 416 staged rows, four waves).
  AttnArgs e = a;
  if (a.hw_exp && a.T - 1 < a.window) e.window = a.window - 32 * ((a.window - (a.T - 1)) / 32);
  if (a.head_dim == 64) pick_nch<64>(b, e);
  else pick_nch<32>(b, e);
}

}  // namespace pf
