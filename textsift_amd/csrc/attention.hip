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
#include "common.cuh"
#include "epilogue.cuh"
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

// NW waves x 16 queries per workgroup; NCH 32-key chunks per 16-query tile.
// HWX: the softmax exponentials use the hardware exp2 (v_exp_f32, about 1
// ulp) on scores pre-multiplied by log2(e), as the reference's GPU shader
// uses the WGSL exp (src/native/shaders/banded_attention.wgsl:100-113);
// otherwise they follow the WASM path (polynomial expApprox for the 4-lane
// part, libm exp for the scalar tail). HWX also stores the output with the
// hardware fp16 conversion (subnormals kept) as the shader's f16 store does.
template <int HD, int NCH, int NW, bool HWX>
__global__ __launch_bounds__(64 * NW) void k_banded_attention(AttnArgs a) {
  constexpr int QB = 16 * NW;                // query tokens per workgroup
  constexpr int ROWS = 16 * (NW - 1) + 32 * NCH;  // staged key rows (every wave's chunks)
  constexpr int LDK = HD + 8;                // K row stride (halves)
  constexpr int LDV = ROWS + 8;              // V^T row stride (halves)
  constexpr int NDH = HD / 32;               // MFMA K-steps over head_dim for Q.K
  constexpr int NDT = HD / 16;               // 16-row dim tiles of O^T
  static_assert(ROWS % 4 == 0, "V^T staging writes 4 keys at a time");
  extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
  _Float16* Ks = smem;                       // [ROWS][LDK]
  _Float16* Vt = smem + ROWS * LDK;          // [HD][LDV]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int t0 = blockIdx.x * QB;
  const int g = blockIdx.y;                  // kv head
  const int bseq = blockIdx.z;
  const int T = a.T, W = a.window;
  const size_t seq0 = (size_t)bseq * T;
  const int kbase = t0 - W;                  // key index of staged row 0

  // ---- stage K (row-major) and V^T; rows outside [0, T) are zero (masked later)
  for (int i = tid; i < ROWS * (HD / 8); i += 64 * NW) {
    const int r = i / (HD / 8), c = i % (HD / 8);
    const int key = kbase + r;
    u4_t kv = {0u, 0u, 0u, 0u};
    if (key >= 0 && key < T) kv = *reinterpret_cast<const u4_t*>(a.k + (seq0 + key) * a.k_stride + g * HD + c * 8);
    *reinterpret_cast<u4_t*>(&Ks[r * LDK + c * 8]) = kv;
  }
  for (int i = tid; i < (ROWS / 4) * (HD / 8); i += 64 * NW) {  // 4 keys x 8 dims per thread
    const int r4 = (i / (HD / 8)) * 4, c = i % (HD / 8);
    h8_t vh[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int key = kbase + r4 + u;
      u4_t vv = {0u, 0u, 0u, 0u};
      if (key >= 0 && key < T) vv = *reinterpret_cast<const u4_t*>(a.v + (seq0 + key) * a.v_stride + g * HD + c * 8);
      vh[u] = __builtin_bit_cast(h8_t, vv);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<h4_t*>(&Vt[(c * 8 + j) * LDV + r4]) = h4_t{vh[0][j], vh[1][j], vh[2][j], vh[3][j]};
  }
  __syncthreads();

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
  constexpr float LOG2_E = 1.44269504088896340736f;
  const float sscale = HWX ? a.scale * LOG2_E : a.scale;  // scores in the exponent's units

  for (int hh = 0; hh < G; ++hh) {
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
    const float sink = a.sinks ? (HWX ? a.sinks[hq] * LOG2_E : a.sinks[hq]) : -INFINITY;

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
                         (HWX || !(32 * c + 32 > tail_lo && 32 * c < any_hi));
      if (plain) {  // wave-uniform: every slot in every window, no tail key
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float e = HWX ? __builtin_amdgcn_exp2f(s[c][kt][r] - m) : exp_approx_fast(s[c][kt][r] - m);
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
            float e = HWX ? __builtin_amdgcn_exp2f(x) : (off >= tail ? expf(x) : exp_approx_fast(x));
            e = (sv != sv) ? 0.0f : e;
            s[c][kt][r] = e;
            l += e;
          }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if constexpr (HWX) l += __builtin_amdgcn_exp2f(sink - m);
    else l += n_keys < vec_end ? exp_approx_fast(sink - m) : expf(sink - m);
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
        *reinterpret_cast<u2_t*>(orow + 16 * dt + 4 * lg) = HWX ? to_f16x4_native(ov) : to_f16x4(ov);
      }
    }
  }
}

template <int HD, int NCH, int NW, bool HWX>
void launch_attn_x(pfhip_backend* b, const AttnArgs& a) {
  constexpr int ROWS = 16 * (NW - 1) + 32 * NCH;
  const size_t lds = (size_t)(ROWS * (HD + 8) + HD * (ROWS + 8)) * sizeof(_Float16);
  static bool attr_set = false;
  if (!attr_set) {
    PF_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_banded_attention<HD, NCH, NW, HWX>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr_set = true;
  }
  dim3 grid((a.T + 16 * NW - 1) / (16 * NW), a.Hkv, a.B);
  ProfScope ps(b, "banded_attention");
  hipLaunchKernelGGL((k_banded_attention<HD, NCH, NW, HWX>), grid, dim3(64 * NW), lds, b->stream, a);
  PF_HIP(hipGetLastError());
}

template <int HD, int NCH, int NW>
void launch_attn(pfhip_backend* b, const AttnArgs& a) {
  if (a.hw_exp) launch_attn_x<HD, NCH, NW, true>(b, a);
  else launch_attn_x<HD, NCH, NW, false>(b, a);
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
  PF_CHECK(a.q_stride % 8 == 0 && a.k_stride % 8 == 0 && a.v_stride % 8 == 0 && a.out_stride % 4 == 0,
           "banded_attention: row strides must allow 16-byte loads");
  PF_CHECK(((uintptr_t)a.q & 15) == 0 && ((uintptr_t)a.k & 15) == 0 && ((uintptr_t)a.v & 15) == 0 &&
               ((uintptr_t)a.out & 7) == 0,
           "banded_attention: operands must be 16-byte aligned");
  if (a.B <= 0 || a.T <= 0) return;
  if (a.head_dim == 64) pick_nch<64>(b, a);
  else pick_nch<32>(b, a);
}

}  // namespace pf
