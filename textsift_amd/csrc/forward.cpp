// forward.cpp — the privacy-filter encoder forward on one GPU
// (include/pfhip.h: pfhip_model_*).
//
// Composition follows the reference's WASM path (browser/inference/
// model.ts:50-105, block.ts:108-197, attention.ts:45-215, expert.ts:104-212)
// with the GPU decomposition of NodeBackend.forward
// (native/backend.ts:433-704) collapsed into 11 launches per layer:
//
//   [layer 0 only] embed -> h ; rms_norm(h, ln_in) -> xn (f32 as hi/lo fp16 planes)
//   per layer l:
//     QKV GEMM  xn -> qkv (fp16, bias, RoPE on q/k in the epilogue)
//     banded attention qkv -> att (fp16)
//     O GEMM    att -> o (fp16)
//     add+rms_norm  h + o -> h2 (fp16), xn (hi/lo)
//     router GEMM xn -> logits (f32); top-k/softmax -> (idx, w)
//     routing plan: count / scan / scatter (stable counting sort by expert)
//     gate_up grouped GEMM (gathered xn rows) + SwiGLU -> glu (f32 as hi/lo)
//     down grouped GEMM glu -> y (f32, slot order)
//     combine: h_next = fp16(h2 + fp16(sum_k w_k y_k)) ; xn = rms_norm(h_next, next ln)
//   classifier GEMM xn -> fp16 logits -> f32
//
// B sequences of T tokens are processed together: every token-wise kernel
// sees B*T rows; attention bands never cross a sequence boundary; RoPE
// positions restart per sequence. Weights stay in the ONNX byte layouts;
// finalize() concatenates q/k/v into one [1152][K] weight so the three
// projections are one GEMM.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "pfhip_internal.h"

using namespace pf;

namespace pf {
// Expert tile rows for the grouped GEMMs, from the mean rows per expert:
// 128 from 256 on, 64 below, 16 (the all-K tile, fp16 numerics, K = 640 or
// 896) below 32; fragments per wave 4, 5 and 1 respectively.
ExpertTile expert_tile(int M, int topk, int experts, bool fp16, int D, int F) {
  const int per_expert = (int)((long)M * topk / experts);
  if (per_expert >= 256) return {128, 4};
  const auto small_k = [](int k) { return k == 640 || k == 896; };
  if (fp16 && small_k(D) && small_k(F) && per_expert < 32) return {16, 1};
  return {64, 5};
}
}  // namespace pf

namespace {

struct DevT {
  void* p = nullptr;
  size_t n = 0;
};

struct QW {  // one MatMulNBits weight on device
  const uint8_t* q = nullptr;
  const uint16_t* s = nullptr;
  const uint8_t* z = nullptr;
  const uint16_t* bias = nullptr;
};

struct W4 {  // one weight in the gemm_w4 form (w4_prepare)
  const uint32_t* w = nullptr;
  const uint32_t* sz = nullptr;
};

struct LayerW {
  const uint16_t* ln_in;
  const uint16_t* ln_post;
  QW qkv, o, router, gate_up, down;
  W4 qkv4, o4, router4, gate_up4, down4;  // PFHIP_PRECISION_FP16 only
  const float* sinks;
};

// ONNX-layout byte sizes of a MatMulNBits weight [N][K]
size_t q_bytes(size_t N, size_t K) { return N * K / 2; }
size_t s_bytes(size_t N, size_t K) { return N * (K / 32) * 2; }
size_t z_bytes(size_t N, size_t K) { return N * ((K / 32 + 1) / 2); }

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

// Copies on the backend's stream, waited for: the stream is non-blocking, so
// copies on the null stream would not be ordered before its kernels (a
// pageable host -> device hipMemcpy may return before its DMA has landed).
void copy_sync(pfhip_backend* b, void* dst, const void* src, size_t n, hipMemcpyKind kind) {
  PF_HIP(hipMemcpyAsync(dst, src, n, kind, b->stream));
  PF_HIP(hipStreamSynchronize(b->stream));
}

}  // namespace

// One captured forward: the launches of run_forward for one (batch,
// seq_len) on fixed ids / mask / logits buffers, the model's scratch and RoPE
// tables. An entry without exec has run once eagerly: the first call of a
// shape grows the scratch and tables and sets the kernels' attributes, none
// of which a capture may contain; the second is captured and replayed.
struct FwdGraph {
  int B = 0, T = 0;
  const void* ids = nullptr;
  const void* mask = nullptr;
  void* logits = nullptr;
  hipGraphExec_t exec = nullptr;
};

struct pfhip_model {
  pfhip_backend* b = nullptr;
  pfhip_model_config cfg{};
  std::map<std::string, size_t> expected;   // name -> byte size
  std::map<std::string, DevT> w;            // uploaded tensors
  std::vector<DevT> owned;                  // derived tensors (fused qkv)
  std::vector<LayerW> layers;
  W4 score4;
  bool finalized = false;
  // per-forward scratch
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  // RoPE tables for one sequence length
  int rope_T = 0;
  float* rope_cos = nullptr;  // fp16 table entries, widened as the reference widens them
  float* rope_sin = nullptr;
  uint16_t* rope_pairs = nullptr;  // [T][hd/2][cos, sin] fp16 bits (fp16 numerics)
  // host-API staging
  pfhip_buffer* ids_buf = nullptr;
  pfhip_buffer* mask_buf = nullptr;
  pfhip_buffer* logits_buf = nullptr;
  // debug taps (not recorded by the allocation-free entry)
  bool taps = false;
  bool in_noalloc = false;
  std::map<std::string, std::vector<uint8_t>> tap;
  // HIP graphs of the device-resident forward, one per (batch, seq_len,
  // buffers): the reference records a forward's whole dispatch sequence into
  // one encoder and submits it once (native/backend.ts:485,693)
  bool graphs = true;
  std::vector<FwdGraph> graph_cache;
};

namespace {

void expect(pfhip_model* m, const std::string& name, size_t bytes) { m->expected[name] = bytes; }

void expect_qw(pfhip_model* m, const std::string& p, size_t N, size_t K, size_t lead = 1) {
  expect(m, p + ".int4", lead * q_bytes(N, K));
  expect(m, p + ".scales", lead * s_bytes(N, K));
  expect(m, p + ".zp", lead * z_bytes(N, K));
  expect(m, p + ".bias", lead * N * 2);
}

template <class T>
const T* W(pfhip_model* m, const std::string& name) {
  auto it = m->w.find(name);
  if (it == m->w.end()) throw Error("missing weight \"" + name + "\"");
  return static_cast<const T*>(it->second.p);
}

QW qw(pfhip_model* m, const std::string& p) {
  return QW{W<uint8_t>(m, p + ".int4"), W<uint16_t>(m, p + ".scales"), W<uint8_t>(m, p + ".zp"),
            W<uint16_t>(m, p + ".bias")};
}

// Scale-folded copy of a MatMulNBits weight ([lead][N][K]) for gemm_w4.
W4 prepare_w4(pfhip_model* m, const QW& q, size_t N, size_t K, size_t lead = 1) {
  DevT tw, ts;
  PF_HIP(hipMalloc(&tw.p, lead * N * K / 2));
  m->owned.push_back(tw);
  PF_HIP(hipMalloc(&ts.p, lead * N * (K / 32) * 4));
  m->owned.push_back(ts);
  w4_prepare(m->b, q.q, q.s, q.z, static_cast<uint32_t*>(tw.p), static_cast<uint32_t*>(ts.p), (int)(lead * N),
             (int)K);
  return W4{static_cast<const uint32_t*>(tw.p), static_cast<const uint32_t*>(ts.p)};
}

// YARN RoPE tables (browser/inference/rope.ts:27-144): inverse frequencies
// in f32 from float64 math, angle = t * invFreq in float64, cos/sin scaled by
// 0.1 ln(factor) + 1, stored to f32 and then to fp16 (rope.ts:82-108).
uint16_t f32_to_fp16_host(float f) {
  if (f == 0.0f) return 0;
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u, exp32 = (u >> 23) & 0xffu, mant = u & 0x7fffffu;
  if (exp32 == 0xffu) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
  int e16 = (int)exp32 - 127 + 15;
  if (e16 >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (e16 <= 0) {
    if (e16 < -10) return (uint16_t)sign;
    const uint32_t shift = (uint32_t)(14 - e16), m24 = mant | 0x800000u;
    return (uint16_t)(sign | ((m24 + (1u << (shift - 1))) >> shift));
  }
  const uint32_t lsb = (mant >> 13) & 1u;
  uint32_t m10 = (mant + 0xfffu + lsb) >> 13;
  uint32_t e = (uint32_t)e16;
  if (m10 >= 0x400u) {
    m10 = 0;
    if (++e >= 0x1fu) return (uint16_t)(sign | 0x7c00u);
  }
  return (uint16_t)(sign | (e << 10) | m10);
}

// fp16 bits -> f32 as zig/math.zig:45-52 widens (subnormals rebiased).
float wasm_h2f_host(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16, rest = (uint32_t)h & 0x7fffu;
  const uint32_t u = sign | (rest == 0u ? 0u : (rest << 13) + (112u << 23));
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void build_rope_tables(const pfhip_model_config& c, int T, std::vector<uint16_t>& cs, std::vector<uint16_t>& sn) {
  const int hd = (int)c.head_dim, half = hd / 2;
  std::vector<float> ex(half), in(half), inv(half);
  for (int i = 0; i < half; ++i) {
    const double pos = std::pow(c.rope_theta, (double)(2 * i) / (double)hd);
    ex[i] = (float)(1.0 / pos);
    in[i] = (float)(1.0 / (c.rope_factor * pos));
  }
  const double PI = 3.141592653589793;
  double lo = ((double)hd * std::log((double)c.rope_orig_max / (c.rope_beta_fast * 2.0 * PI))) /
              (2.0 * std::log(c.rope_theta));
  double hi = ((double)hd * std::log((double)c.rope_orig_max / (c.rope_beta_slow * 2.0 * PI))) /
              (2.0 * std::log(c.rope_theta));
  if (c.rope_truncate) {
    lo = std::floor(lo);
    hi = std::ceil(hi);
  }
  lo = std::max(lo, 0.0);
  hi = std::min(hi, (double)(hd - 1));
  const double rmax = hi == lo ? lo + 0.001 : hi;
  for (int i = 0; i < half; ++i) {
    const double lin = ((double)i - lo) / (rmax - lo);
    const double ramp = std::min(std::max(lin, 0.0), 1.0);
    const double ef = 1.0 - ramp;
    inv[i] = (float)((double)in[i] * (1.0 - ef) + (double)ex[i] * ef);
  }
  const double scaling = c.rope_factor <= 1.0 ? 1.0 : 0.1 * std::log(c.rope_factor) + 1.0;
  cs.resize((size_t)T * half);
  sn.resize((size_t)T * half);
  for (int t = 0; t < T; ++t)
    for (int i = 0; i < half; ++i) {
      const double ang = (double)t * (double)inv[i];
      cs[(size_t)t * half + i] = f32_to_fp16_host((float)(std::cos(ang) * scaling));
      sn[(size_t)t * half + i] = f32_to_fp16_host((float)(std::sin(ang) * scaling));
    }
}

// The kernels address activation rows with 32-bit element offsets: every
// [rows][width] array of the forward must hold fewer than 2^31 elements
// (the widest are the routed [M * topk][max(hidden, dff)] expert planes).
// Checked before any scratch is allocated or kernel launched.
void check_row_limits(const pfhip_model_config& c, size_t M) {
  const size_t S = M * c.topk;
  const size_t NQKV = (size_t)(c.heads + 2 * c.kv_heads) * c.head_dim;
  const size_t widest = std::max({M * NQKV, M * c.heads * c.head_dim, M * c.experts, S * c.hidden, S * c.dff,
                                  M * c.classes});
  PF_CHECK(widest < ((size_t)1 << 31),
           "batch * seq_len too large for this model: a [rows][width] activation array of " +
               std::to_string(widest) + " elements exceeds the kernels' 32-bit offsets");
}

struct Scr {
  uint16_t *h0, *h1, *h2, *qkv, *att, *o, *logits16;
  uint16_t *xn_hi, *xn_lo, *glu_hi, *glu_lo;
  float *rlogits, *rw, *y, *logits;
  int32_t* ridx;
  void* plan;
};

// The 16-token GEMM tile loads all of K (640 or 896) at once: a workgroup
// waits on memory once instead of once per 128-wide K chunk, which is what
// a GEMM of a few workgroups costs. fp16 numerics only.
constexpr int SMALL_M = 2048;           // dense GEMMs: rows up to this
bool small_k(size_t K) { return K == 640 || K == 896; }

int tile_for(const pfhip_model_config& c, int M) {
  return expert_tile(M, (int)c.topk, (int)c.experts, c.precision == PFHIP_PRECISION_FP16, (int)c.hidden,
                     (int)c.dff)
      .t;
}

size_t scratch_layout(const pfhip_model_config& c, int M, Scr* s, void* base) {
  const size_t D = c.hidden, E = c.experts, K = c.topk, F = c.dff, C = c.classes;
  const size_t NQKV = (size_t)(c.heads + 2 * c.kv_heads) * c.head_dim;
  const size_t HQ = (size_t)c.heads * c.head_dim;
  const size_t S = (size_t)M * K;
  const int tt = tile_for(c, M);
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) -> void* {
    void* r = p ? p + off : nullptr;
    off += al256(bytes);
    return r;
  };
  Scr t;
  t.h0 = (uint16_t*)take((size_t)M * D * 2);
  t.h1 = (uint16_t*)take((size_t)M * D * 2);
  t.h2 = (uint16_t*)take((size_t)M * D * 2);
  t.xn_hi = (uint16_t*)take((size_t)M * D * 2);
  t.xn_lo = (uint16_t*)take((size_t)M * D * 2);
  t.qkv = (uint16_t*)take((size_t)M * NQKV * 2);
  t.att = (uint16_t*)take((size_t)M * HQ * 2);
  t.o = (uint16_t*)take((size_t)M * D * 2);
  t.rlogits = (float*)take((size_t)M * E * 4);
  t.ridx = (int32_t*)take(S * 4);
  t.rw = (float*)take(S * 4);
  t.glu_hi = (uint16_t*)take(S * F * 2);
  t.glu_lo = (uint16_t*)take(S * F * 2);
  t.y = (float*)take(S * D * (c.precision == PFHIP_PRECISION_FP16 ? 2 : 4));  // fp16 in the fp16 numerics
  t.logits16 = (uint16_t*)take((size_t)M * C * 2);
  t.logits = (float*)take((size_t)M * C * 4);
  t.plan = take(moe_plan_bytes(M, (int)K, (int)E, tt));
  if (s) *s = t;
  return off;
}

}  // namespace

namespace pf {
void cast_f16_f32_ieee(pfhip_backend* b, const uint16_t* s, float* d, size_t n);
}

static void record_tap(pfhip_model* m, const std::string& name, const void* dev, size_t bytes) {
  if (!m->taps || m->in_noalloc) return;
  std::vector<uint8_t>& v = m->tap[name];
  v.resize(bytes);
  PF_HIP(hipMemcpyAsync(v.data(), dev, bytes, hipMemcpyDeviceToHost, m->b->stream));
  PF_HIP(hipStreamSynchronize(m->b->stream));
}

// Drops every captured forward (their launches name the scratch, tables
// and weights of the moment they were captured).
static void clear_graphs(pfhip_model* m) {
  for (auto& g : m->graph_cache)
    if (g.exec) hipGraphExecDestroy(g.exec);
  m->graph_cache.clear();
}

// Host-built YARN tables for T positions, replacing smaller ones.
static void ensure_rope(pfhip_model* m, int T) {
  pfhip_backend* b = m->b;
  std::vector<uint16_t> cs, sn;
  build_rope_tables(m->cfg, T, cs, sn);
  clear_graphs(m);
  if (m->rope_cos) {
    PF_HIP(hipStreamSynchronize(b->stream));
    hipFree(m->rope_cos);
    hipFree(m->rope_sin);
    hipFree(m->rope_pairs);
    m->rope_cos = m->rope_sin = nullptr;
    m->rope_pairs = nullptr;
    m->rope_T = 0;
  }
  std::vector<float> csf(cs.size()), snf(sn.size());
  std::vector<uint16_t> pairs(2 * cs.size());
  for (size_t i = 0; i < cs.size(); ++i) {
    csf[i] = wasm_h2f_host(cs[i]);
    snf[i] = wasm_h2f_host(sn[i]);
    pairs[2 * i] = cs[i];
    pairs[2 * i + 1] = sn[i];
  }
  PF_HIP(hipMalloc(&m->rope_cos, csf.size() * 4));
  PF_HIP(hipMalloc(&m->rope_sin, snf.size() * 4));
  PF_HIP(hipMalloc(&m->rope_pairs, pairs.size() * 2));
  copy_sync(b, m->rope_cos, csf.data(), csf.size() * 4, hipMemcpyHostToDevice);
  copy_sync(b, m->rope_sin, snf.data(), snf.size() * 4, hipMemcpyHostToDevice);
  copy_sync(b, m->rope_pairs, pairs.data(), pairs.size() * 2, hipMemcpyHostToDevice);
  m->rope_T = T;
}

// fixed_scratch: the allocation-free entry's scratch (nothing is allocated
// and no taps are recorded); NULL: the model's own, grown as needed.
static void run_forward(pfhip_model* m, const int32_t* ids, const uint8_t* mask, int B, int T, float* logits_out,
                        void* fixed_scratch = nullptr) {
  pfhip_backend* b = m->b;
  const pfhip_model_config& c = m->cfg;
  const int M = B * T;
  const int D = (int)c.hidden, E = (int)c.experts, K = (int)c.topk, F = (int)c.dff, C = (int)c.classes;
  const int Hq = (int)c.heads, Hkv = (int)c.kv_heads, hd = (int)c.head_dim;
  const int NQKV = (Hq + 2 * Hkv) * hd;
  const int tt = tile_for(c, M);

  // scratch (the layout's size is not monotonic in M: the expert tile list
  // of a smaller M on a smaller tile can be longer)
  const size_t bytes = scratch_layout(c, M, nullptr, nullptr);
  void* base = fixed_scratch;
  if (fixed_scratch) {
    PF_CHECK(bytes <= NOALLOC_SCRATCH_BYTES, "batch * seq_len = " + std::to_string(M) + " needs " +
                                                 std::to_string(bytes) + " bytes of scratch, more than the " +
                                                 std::to_string(NOALLOC_SCRATCH_BYTES) +
                                                 " of the allocation-free forward");
  } else if (bytes > m->scratch_bytes) {
    clear_graphs(m);
    if (m->scratch) {
      PF_HIP(hipStreamSynchronize(b->stream));
      PF_HIP(hipFree(m->scratch));
      m->scratch = nullptr;
    }
    PF_HIP(hipMalloc(&m->scratch, bytes));
    m->scratch_bytes = bytes;
  }
  if (!base) base = m->scratch;
  Scr s;
  scratch_layout(c, M, &s, base);
  MoePlan plan = moe_plan_carve(s.plan, M, K, E, tt);

  // RoPE tables: built on the host for at least T positions (row t depends
  // on t alone, so tables built for more positions serve any shorter T)
  if (m->rope_T < T) {
    PF_CHECK(!fixed_scratch, "seq_len exceeds the RoPE tables already built (the allocation-free forward "
                             "cannot build longer ones)");
    ensure_rope(m, T);
  }

  const bool f16 = c.precision == PFHIP_PRECISION_FP16;
  // GEMM tiles of the fp16 path: (tokens, 16-row fragments per wave)
  const int gw_t = tt, gw_f = expert_tile(M, K, E, f16, D, F).wf;
  // dense GEMMs of at most SMALL_M rows (O and the classifier 2x, the
  // router 8x: measured crossovers) take the all-K 16-token tile
  auto small_dense = [&](int k, int limit = SMALL_M) { return M <= limit && small_k((size_t)k); };
  // O projection: one kernel with the add + norm from 16384 rows; below, the
  // O GEMM, and the add + norm either in the router GEMM (its 16-token tile
  // holds whole 640-wide rows) or as its own kernel
  const bool fused_o = f16 && D == 640 && (Hq * hd == 640 || Hq * hd == 896) && M >= 16384;
  const bool norm_in_router = f16 && !fused_o && D == 640 && small_dense(D, 8 * SMALL_M);
  // fp16 numerics with the model's 128 experts and top-4: the router GEMM's
  // epilogue selects the experts (bit-identical to router_topk) and, above
  // one counting block of tokens, counts each router tile's rows per expert,
  // from which one kernel builds the routing plan
  const bool fused_topk = f16 && E == 128 && K == 4;
  const int router_tile = small_dense(D, 8 * SMALL_M) ? 16 : 64;
  const bool route_counts = fused_topk && M > 1024;
  // up to 16 rows the router is one workgroup, which then also builds the
  // routing plan (no separate plan kernel: one launch fewer per layer)
  const bool plan_in_router = fused_topk && router_tile == 16 && M <= 16;

  if (f16) {
    embed_rms_norm_f16(b, W<uint8_t>(m, "embed.int4"), W<uint16_t>(m, "embed.scales"), W<uint8_t>(m, "embed.zp"), ids,
                       m->layers[0].ln_in, s.h0, s.xn_hi, M, (int)c.vocab, D, c.eps);
  } else {
    embed_lookup(b, W<uint8_t>(m, "embed.int4"), W<uint16_t>(m, "embed.scales"), W<uint8_t>(m, "embed.zp"), ids, s.h0,
                 M, (int)c.vocab, D);
    rms_norm_split(b, s.h0, m->layers[0].ln_in, s.xn_hi, s.xn_lo, M, D, c.eps);
  }
  record_tap(m, "embed", s.h0, (size_t)M * D * 2);
  record_tap(m, "xn0", s.xn_hi, (size_t)M * D * 2);
  uint16_t* h = s.h0;
  uint16_t* hn = s.h1;
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const LayerW& L = m->layers[l];
    const std::string tag = std::to_string(l);
    {  // QKV (+bias, RoPE)
      GemmArgs a;
      a.x = s.xn_hi; a.x_lo = s.xn_lo; a.ldx = D;
      a.w = L.qkv.q; a.ws = L.qkv.s; a.wz = L.qkv.z; a.bias = L.qkv.bias;
      a.out = s.qkv; a.ldo = NQKV; a.M = M; a.N = NQKV; a.K = D;
      a.rope_cos = m->rope_cos; a.rope_sin = m->rope_sin; a.rope_pairs = m->rope_pairs;
      a.seq_len = T; a.rope_cols = (Hq + Hkv) * hd;
      if (f16) {
        a.w = reinterpret_cast<const uint8_t*>(L.qkv4.w); a.wsz = L.qkv4.sz;
        const bool sm = small_dense(D);
        gemm_w4(b, a, XKind::F16, Epi::ROPE_F16, false, sm ? 16 : 128, sm ? 1 : 4, "gemm_qkv_rope");
      } else {
        gemm_int4(b, a, XKind::SPLIT, Epi::ROPE_F16, false, 128, "gemm_qkv_rope");
      }
    }
    record_tap(m, "qkv." + tag, s.qkv, (size_t)M * NQKV * 2);
    {
      AttnArgs a{};
      a.q = s.qkv; a.q_stride = NQKV;
      a.k = s.qkv + Hq * hd; a.k_stride = NQKV;
      a.v = s.qkv + (Hq + Hkv) * hd; a.v_stride = NQKV;
      a.sinks = L.sinks; a.mask = mask;
      a.out = s.att; a.out_stride = Hq * hd;
      a.B = B; a.T = T; a.Hq = Hq; a.Hkv = Hkv; a.head_dim = hd; a.window = (int)c.window; a.scale = 1.0f;
      a.hw_exp = f16;
      banded_attention(b, a);
    }
    record_tap(m, "att." + tag, s.att, (size_t)M * Hq * hd * 2);
    {
      GemmArgs a;
      a.x = s.att; a.ldx = Hq * hd;
      a.w = L.o.q; a.ws = L.o.s; a.wz = L.o.z; a.bias = L.o.bias;
      a.out = s.o; a.ldo = D; a.M = M; a.N = D; a.K = Hq * hd;
      if (f16) {
        a.w = reinterpret_cast<const uint8_t*>(L.o4.w); a.wsz = L.o4.sz;
        // whole rows per workgroup with the add + norm fused: one 64-row tile
        // per CU and latency-bound, so it pays only once there are enough
        // rows to fill the chip (measured: 87 vs 97 us at 32768 rows; 44 vs
        // 40 us at 8192 and 40 vs 31 us at 64 for the two-kernel form)
        if (fused_o) {
          gemm_w4_add_rmsnorm(b, a, h, L.ln_post, s.h2, s.xn_hi, c.eps);
        } else {
          const bool sm = small_dense(Hq * hd, 2 * SMALL_M);
          gemm_w4(b, a, XKind::F16, Epi::F16, false, sm ? 16 : 128, sm ? 1 : 4, "gemm_o");
          if (!norm_in_router) add_rms_norm_f16(b, h, s.o, L.ln_post, s.h2, s.xn_hi, M, D, c.eps);
        }
      } else {
        gemm_int4(b, a, XKind::F16, Epi::F16, false, 128, "gemm_o");
        add_rms_norm_split(b, h, s.o, L.ln_post, s.h2, s.xn_hi, s.xn_lo, M, D, c.eps);
      }
    }
    {
      GemmArgs a;
      a.x = s.xn_hi; a.x_lo = s.xn_lo; a.ldx = D;
      if (norm_in_router) {  // the post-attention add + norm on the router's way in
        a.x = s.o;
        a.nrm_res = h; a.nrm_gamma = L.ln_post; a.nrm_h = s.h2; a.nrm_xn = s.xn_hi; a.nrm_eps = c.eps;
      }
      a.w = L.router.q; a.ws = L.router.s; a.wz = L.router.z; a.bias = L.router.bias;
      a.out = s.rlogits; a.ldo = E; a.M = M; a.N = E; a.K = D;
      if (f16) {
        a.w = reinterpret_cast<const uint8_t*>(L.router4.w); a.wsz = L.router4.sz;
        if (fused_topk) {
          a.topk_idx = s.ridx; a.topk_w = s.rw; a.topk_k = K; a.topk_wscale = 1.0f;
          if (route_counts) a.topk_counts = plan.tile_counts;  // per router tile: the routing plan's counts
          if (plan_in_router) {
            a.plan_expert_off = plan.expert_off; a.plan_slot_token = plan.slot_token; a.plan_slot_of = plan.slot_of;
            a.plan_tiles = plan.tiles; a.plan_num_tiles = plan.num_tiles; a.plan_tile_t = plan.tile_t;
          }
          if (!m->taps) a.out = nullptr;  // the logits stay in LDS (written only for the debug taps)
        }
        gemm_w4(b, a, XKind::F16, fused_topk ? Epi::F32_TOPK : Epi::F32, false, router_tile, 2, "gemm_router");
      } else {
        gemm_int4(b, a, XKind::SPLIT, Epi::F32, false, 128, "gemm_router");
      }
      if (!fused_topk) router_topk(b, s.rlogits, s.ridx, s.rw, M, E, K, 1.0f);
    }
    record_tap(m, "h2." + tag, s.h2, (size_t)M * D * 2);
    record_tap(m, "xn2." + tag, s.xn_hi, (size_t)M * D * 2);
    record_tap(m, "router." + tag, s.rlogits, (size_t)M * E * 4);
    record_tap(m, "ridx." + tag, s.ridx, (size_t)M * K * 4);
    record_tap(m, "rw." + tag, s.rw, (size_t)M * K * 4);
    if (route_counts) {
      record_tap(m, "rcount." + tag, plan.tile_counts, (size_t)((M + router_tile - 1) / router_tile) * E * 4);
      moe_route_counts(b, s.ridx, plan.tile_counts, router_tile, M, K, E, plan);
    } else if (!plan_in_router) {
      moe_route(b, s.ridx, M, K, E, plan);
    }
    record_tap(m, "expert_off." + tag, plan.expert_off, (size_t)(E + 1) * 4);
    record_tap(m, "slot_token." + tag, plan.slot_token, (size_t)M * K * 4);
    record_tap(m, "slot_of." + tag, plan.slot_of, (size_t)M * K * 4);
    {
      GemmArgs g;
      g.x = s.xn_hi; g.x_lo = s.xn_lo; g.ldx = D; g.row_map = plan.slot_token;
      g.w = L.gate_up.q; g.ws = L.gate_up.s; g.wz = L.gate_up.z; g.bias = L.gate_up.bias;
      g.w_gs = q_bytes(2 * F, D); g.ws_gs = s_bytes(2 * F, D) / 2; g.wz_gs = z_bytes(2 * F, D);
      g.bias_gs = (size_t)2 * F;
      g.out = s.glu_hi; g.out_lo = s.glu_lo; g.ldo = F; g.M = M * K; g.N = 2 * F; g.K = D;
      g.tiles = plan.tiles; g.num_tiles = plan.num_tiles; g.max_tiles = plan.max_tiles;
      if (f16) {
        g.w = reinterpret_cast<const uint8_t*>(L.gate_up4.w); g.wsz = L.gate_up4.sz;
        g.wsz_gs = (size_t)2 * F * (D / 32);
        gemm_w4(b, g, XKind::F16, Epi::SWIGLU_F16, true, gw_t, gw_f, "gemm_moe_gate_up");
      } else {
        gemm_int4(b, g, XKind::SPLIT, Epi::SWIGLU_SPLIT, true, tt, "gemm_moe_gate_up");
      }
    }
    {
      GemmArgs d;
      d.x = s.glu_hi; d.x_lo = s.glu_lo; d.ldx = F;
      d.w = L.down.q; d.ws = L.down.s; d.wz = L.down.z; d.bias = L.down.bias;
      d.w_gs = q_bytes(D, F); d.ws_gs = s_bytes(D, F) / 2; d.wz_gs = z_bytes(D, F); d.bias_gs = (size_t)D;
      d.out = s.y; d.ldo = D; d.M = M * K; d.N = D; d.K = F;
      d.tiles = plan.tiles; d.num_tiles = plan.num_tiles; d.max_tiles = plan.max_tiles;
      if (f16) {
        d.w = reinterpret_cast<const uint8_t*>(L.down4.w); d.wsz = L.down4.sz;
        d.wsz_gs = (size_t)D * (F / 32);
        // fp16 expert outputs (one rounding each; the combine widens them)
        gemm_w4(b, d, XKind::F16, Epi::F16, true, gw_t, gw_f, "gemm_moe_down");
      } else {
        gemm_int4(b, d, XKind::SPLIT, Epi::F32, true, tt, "gemm_moe_down");
      }
    }
    const uint16_t* gamma_next = l + 1 < m->layers.size() ? m->layers[l + 1].ln_in : W<uint16_t>(m, "final_norm");
    moe_combine_norm(b, s.ridx, s.rw, plan.slot_of, s.y, f16, s.h2, hn, gamma_next, s.xn_hi, f16 ? nullptr : s.xn_lo,
                     M, K, D, c.eps);
    record_tap(m, "h." + tag, hn, (size_t)M * D * 2);
    std::swap(h, hn);
  }
  {
    GemmArgs a;
    a.x = s.xn_hi; a.x_lo = s.xn_lo; a.ldx = D;
    QW sc = qw(m, "score");
    a.w = sc.q; a.ws = sc.s; a.wz = sc.z; a.bias = sc.bias;
    a.out = s.logits16; a.ldo = C; a.M = M; a.N = C; a.K = D;
    if (f16) {
      a.w = reinterpret_cast<const uint8_t*>(m->score4.w); a.wsz = m->score4.sz;
      // wasm.ts:776-796 widens the fp16 logits IEEE-correctly: the epilogue
      // stores them widened (the fp16 copy only for the taps)
      a.out_f32w = logits_out ? logits_out : s.logits;
      if (!m->taps) a.out = nullptr;
      gemm_w4(b, a, XKind::F16, Epi::F16, false, small_dense(D, 2 * SMALL_M) ? 16 : 64, 1, "gemm_classifier");
    } else {
      gemm_int4(b, a, XKind::SPLIT, Epi::F16, false, 128, "gemm_classifier");
    }
  }
  record_tap(m, "logits16", s.logits16, (size_t)M * C * 2);
  // wasm.ts:776-796 widens the fp16 logits IEEE-correctly
  if (!f16) cast_f16_f32_ieee(b, s.logits16, logits_out ? logits_out : s.logits, (size_t)M * C);
}

extern "C" {

pfhip_model* pfhip_model_create(pfhip_backend* b, const pfhip_model_config* cfg, char* err, size_t cap) {
  try {
    PF_CHECK(b && cfg, "null argument");
    const pfhip_model_config& c = *cfg;
    PF_CHECK(c.hidden % 32 == 0 && c.dff % 32 == 0 && c.hidden <= 1024, "hidden and dff must be multiples of 32");
    PF_CHECK(c.head_dim == 64, "head_dim must be 64");
    PF_CHECK(c.kv_heads > 0 && c.heads % c.kv_heads == 0, "heads must be a multiple of kv_heads");
    PF_CHECK(c.topk >= 1 && c.topk <= 8 && c.experts >= c.topk && c.experts <= 256, "bad experts / topk");
    PF_CHECK(c.layers >= 1 && c.classes >= 1 && c.vocab >= 1, "bad layers / classes / vocab");
    PF_CHECK(c.window <= 128, "window must be <= 128");
    PF_CHECK(c.precision == PFHIP_PRECISION_FP16 || c.precision == PFHIP_PRECISION_SPLIT, "unknown precision");
    if (c.precision == PFHIP_PRECISION_FP16)
      PF_CHECK(c.hidden % 128 == 0 && c.dff % 128 == 0 && (c.heads * c.head_dim) % 128 == 0,
               "PFHIP_PRECISION_FP16 needs hidden, dff and heads*head_dim to be multiples of 128");
    pfhip_model* m = new pfhip_model();
    m->b = b;
    m->cfg = c;
    const size_t D = c.hidden, Hq = c.heads, Hkv = c.kv_heads, hd = c.head_dim, E = c.experts, F = c.dff;
    expect(m, "embed.int4", q_bytes(c.vocab, D));
    expect(m, "embed.scales", s_bytes(c.vocab, D));
    expect(m, "embed.zp", z_bytes(c.vocab, D));
    for (uint32_t l = 0; l < c.layers; ++l) {
      const std::string p = "layers." + std::to_string(l) + ".";
      expect(m, p + "input_layernorm", D * 2);
      expect(m, p + "post_attention_layernorm", D * 2);
      expect_qw(m, p + "attn.q_proj", Hq * hd, D);
      expect_qw(m, p + "attn.k_proj", Hkv * hd, D);
      expect_qw(m, p + "attn.v_proj", Hkv * hd, D);
      expect_qw(m, p + "attn.o_proj", D, Hq * hd);
      expect(m, p + "attn.sinks", Hq * 4);
      expect_qw(m, p + "router", E, D);
      expect_qw(m, p + "experts.gate_up", 2 * F, D, E);
      expect_qw(m, p + "experts.down", D, F, E);
    }
    expect(m, "final_norm", D * 2);
    expect_qw(m, "score", c.classes, D);
    return m;
  } catch (const std::exception& ex) {
    set_err(err, cap, ex.what());
    return nullptr;
  }
}

void pfhip_model_destroy(pfhip_model* m) {
  if (!m) return;
  hipStreamSynchronize(m->b->stream);
  clear_graphs(m);
  for (auto& kv : m->w) hipFree(kv.second.p);
  for (auto& t : m->owned) hipFree(t.p);
  if (m->scratch) hipFree(m->scratch);
  if (m->rope_cos) hipFree(m->rope_cos);
  if (m->rope_sin) hipFree(m->rope_sin);
  if (m->rope_pairs) hipFree(m->rope_pairs);
  pfhip_release_buffer(m->b, m->ids_buf);
  pfhip_release_buffer(m->b, m->mask_buf);
  pfhip_release_buffer(m->b, m->logits_buf);
  delete m;
}

int pfhip_model_set_weight(pfhip_model* m, const char* name, const void* bytes, size_t n, char* err, size_t cap) {
  try {
    PF_CHECK(m && name && bytes, "null argument");
    auto it = m->expected.find(name);
    PF_CHECK(it != m->expected.end(), std::string("unexpected weight \"") + name + "\"");
    // NodeBackend pads uploads to a multiple of 4 bytes (native/backend.ts:152-160)
    PF_CHECK(n >= it->second && n <= ((it->second + 3) & ~(size_t)3),
             std::string("weight \"") + name + "\" has " + std::to_string(n) + " bytes, expected " +
                 std::to_string(it->second));
    clear_graphs(m);
    auto& t = m->w[name];
    if (t.p && t.n < n) {
      PF_HIP(hipStreamSynchronize(m->b->stream));
      hipFree(t.p);
      t.p = nullptr;
    }
    if (!t.p) PF_HIP(hipMalloc(&t.p, al256(n)));
    t.n = n;
    copy_sync(m->b, t.p, bytes, n, hipMemcpyHostToDevice);
    m->finalized = false;
    return 0;
  } catch (const std::exception& ex) {
    set_err(err, cap, ex.what());
    return -1;
  }
}

int pfhip_model_finalize(pfhip_model* m, char* err, size_t cap) {
  try {
    PF_CHECK(m, "null model");
    for (auto& kv : m->expected)
      PF_CHECK(m->w.count(kv.first), "missing weight \"" + kv.first + "\"");
    const pfhip_model_config& c = m->cfg;
    const size_t D = c.hidden, hd = c.head_dim;
    const size_t Nq = c.heads * hd, Nk = c.kv_heads * hd;
    clear_graphs(m);
    for (auto& t : m->owned) hipFree(t.p);
    m->owned.clear();
    m->layers.clear();
    for (uint32_t l = 0; l < c.layers; ++l) {
      const std::string p = "layers." + std::to_string(l) + ".";
      LayerW L;
      L.ln_in = W<uint16_t>(m, p + "input_layernorm");
      L.ln_post = W<uint16_t>(m, p + "post_attention_layernorm");
      // fused q|k|v weight: rows stacked along N
      DevT fq, fs, fz, fb;
      const size_t N = Nq + 2 * Nk;
      PF_HIP(hipMalloc(&fq.p, q_bytes(N, D)));
      PF_HIP(hipMalloc(&fs.p, s_bytes(N, D)));
      PF_HIP(hipMalloc(&fz.p, z_bytes(N, D)));
      PF_HIP(hipMalloc(&fb.p, N * 2));
      size_t row = 0;
      for (auto& nm : {std::make_pair("q_proj", Nq), std::make_pair("k_proj", Nk), std::make_pair("v_proj", Nk)}) {
        const std::string wp = p + "attn." + nm.first;
        const size_t n = nm.second;
        copy_sync(m->b, (char*)fq.p + q_bytes(row, D), W<uint8_t>(m, wp + ".int4"), q_bytes(n, D),
                  hipMemcpyDeviceToDevice);
        copy_sync(m->b, (char*)fs.p + s_bytes(row, D), W<uint16_t>(m, wp + ".scales"), s_bytes(n, D),
                  hipMemcpyDeviceToDevice);
        copy_sync(m->b, (char*)fz.p + z_bytes(row, D), W<uint8_t>(m, wp + ".zp"), z_bytes(n, D),
                  hipMemcpyDeviceToDevice);
        copy_sync(m->b, (char*)fb.p + row * 2, W<uint16_t>(m, wp + ".bias"), n * 2, hipMemcpyDeviceToDevice);
        row += n;
      }
      m->owned.push_back(fq);
      m->owned.push_back(fs);
      m->owned.push_back(fz);
      m->owned.push_back(fb);
      L.qkv = QW{(const uint8_t*)fq.p, (const uint16_t*)fs.p, (const uint8_t*)fz.p, (const uint16_t*)fb.p};
      L.o = qw(m, p + "attn.o_proj");
      L.router = qw(m, p + "router");
      L.gate_up = qw(m, p + "experts.gate_up");
      L.down = qw(m, p + "experts.down");
      L.sinks = W<float>(m, p + "attn.sinks");
      if (c.precision == PFHIP_PRECISION_FP16) {
        const size_t E = c.experts, F = c.dff;
        L.qkv4 = prepare_w4(m, L.qkv, N, D);
        L.o4 = prepare_w4(m, L.o, D, Nq);
        L.router4 = prepare_w4(m, L.router, E, D);
        L.gate_up4 = prepare_w4(m, L.gate_up, 2 * F, D, E);
        L.down4 = prepare_w4(m, L.down, D, F, E);
      }
      m->layers.push_back(L);
    }
    if (c.precision == PFHIP_PRECISION_FP16) m->score4 = prepare_w4(m, qw(m, "score"), c.classes, D);
    // RoPE tables for one reference chunk (privacy-filter.ts:559: 2048 tokens)
    if (m->rope_T < 2048) ensure_rope(m, 2048);
    PF_HIP(hipStreamSynchronize(m->b->stream));
    m->finalized = true;
    return 0;
  } catch (const std::exception& ex) {
    set_err(err, cap, ex.what());
    return -1;
  }
}

int pfhip_model_enable_taps(pfhip_model* m, int on) {
  if (!m) return -1;
  m->taps = on != 0;
  if (!m->taps) m->tap.clear();
  return 0;
}

int pfhip_model_enable_graphs(pfhip_model* m, int on) {
  if (!m) return -1;
  hipStreamSynchronize(m->b->stream);
  m->graphs = on != 0;
  if (!m->graphs) clear_graphs(m);
  return 0;
}

int pfhip_model_forward_device(pfhip_model* m, pfhip_buffer* ids, pfhip_buffer* mask, uint32_t batch,
                               uint32_t seq_len, pfhip_buffer* logits, char* err, size_t cap) {
  try {
    PF_CHECK(m && ids && logits, "null argument");
    PF_CHECK(batch >= 1 && seq_len >= 1, "batch and seq_len must be positive");
    const size_t M = (size_t)batch * seq_len;
    PF_CHECK(M <= (1u << 22), "batch * seq_len too large");
    check_row_limits(m->cfg, M);
    PF_CHECK(m->finalized, "call pfhip_model_finalize() first");
    PF_CHECK(ids->size >= M * 4, "ids buffer too small");
    PF_CHECK(!mask || mask->size >= M, "mask buffer too small");
    PF_CHECK(logits->size >= M * m->cfg.classes * 4, "logits buffer too small");
    PF_HIP(hipSetDevice(m->b->device));
    const int32_t* idp = static_cast<const int32_t*>(ids->ptr);
    const uint8_t* mkp = mask ? static_cast<const uint8_t*>(mask->ptr) : nullptr;
    float* lgp = static_cast<float*>(logits->ptr);
    if (!m->graphs || m->taps || m->b->profiling) {
      // taps copy to the host mid-forward and profiling brackets launches
      // with events: both run eagerly
      run_forward(m, idp, mkp, (int)batch, (int)seq_len, lgp);
    } else {
      FwdGraph* g = nullptr;
      for (auto& e : m->graph_cache)
        if (e.B == (int)batch && e.T == (int)seq_len && e.ids == idp && e.mask == mkp && e.logits == lgp) g = &e;
      if (!g) {  // first call of this shape: eagerly (it may grow the scratch and tables, which clears the cache)
        run_forward(m, idp, mkp, (int)batch, (int)seq_len, lgp);
        if (m->graph_cache.size() >= 16) {
          if (m->graph_cache.front().exec) hipGraphExecDestroy(m->graph_cache.front().exec);
          m->graph_cache.erase(m->graph_cache.begin());
        }
        FwdGraph e;
        e.B = (int)batch; e.T = (int)seq_len; e.ids = idp; e.mask = mkp; e.logits = lgp;
        m->graph_cache.push_back(e);
      } else {
        if (!g->exec) {  // second call: capture the launches once, then replay them
          hipGraph_t graph = nullptr;
          PF_HIP(hipStreamBeginCapture(m->b->stream, hipStreamCaptureModeRelaxed));
          try {
            run_forward(m, idp, mkp, (int)batch, (int)seq_len, lgp);
          } catch (...) {
            if (hipStreamEndCapture(m->b->stream, &graph) == hipSuccess && graph) hipGraphDestroy(graph);
            throw;
          }
          PF_HIP(hipStreamEndCapture(m->b->stream, &graph));
          const hipError_t ie = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
          hipGraphDestroy(graph);
          PF_HIP(ie);
        }
        PF_HIP(hipGraphLaunch(g->exec, m->b->stream));
      }
    }
    PF_HIP(hipStreamSynchronize(m->b->stream));
    prof_flush(m->b);
    return 0;
  } catch (const std::exception& ex) {
    set_err(err, cap, ex.what());
    return -1;
  }
}

int pfhip_model_forward_device_noalloc(pfhip_model* m, pfhip_buffer* ids, pfhip_buffer* mask, uint32_t batch,
                                       uint32_t seq_len, pfhip_buffer* logits, char* err, size_t cap) {
  try {
    PF_CHECK(m && ids && logits, "null argument");
    PF_CHECK(batch >= 1 && seq_len >= 1, "batch and seq_len must be positive");
    const size_t M = (size_t)batch * seq_len;
    PF_CHECK(M <= (1u << 22), "batch * seq_len too large");
    check_row_limits(m->cfg, M);
    PF_CHECK(m->finalized, "call pfhip_model_finalize() first");
    PF_CHECK(ids->size >= M * 4, "ids buffer too small");
    PF_CHECK(!mask || mask->size >= M, "mask buffer too small");
    PF_CHECK(logits->size >= M * m->cfg.classes * 4, "logits buffer too small");
    PF_HIP(hipSetDevice(m->b->device));
    void* fixed = noalloc_scratch(m->b->device);  // looked up at backend creation; no allocation here
    m->in_noalloc = true;
    try {
      run_forward(m, static_cast<const int32_t*>(ids->ptr), mask ? static_cast<const uint8_t*>(mask->ptr) : nullptr,
                  (int)batch, (int)seq_len, static_cast<float*>(logits->ptr), fixed);
    } catch (...) {
      m->in_noalloc = false;
      throw;
    }
    m->in_noalloc = false;
    PF_HIP(hipStreamSynchronize(m->b->stream));
    prof_flush(m->b);
    return 0;
  } catch (const std::exception& ex) {
    set_err(err, cap, ex.what());
    return -1;
  }
}

int pfhip_model_forward(pfhip_model* m, const int32_t* ids, const uint8_t* mask, uint32_t batch, uint32_t seq_len,
                        float* logits, char* err, size_t cap) {
  try {
    PF_CHECK(m && ids && logits, "null argument");
    PF_CHECK(batch >= 1 && seq_len >= 1, "batch and seq_len must be positive");
    const size_t M = (size_t)batch * seq_len;
    char e2[PFHIP_ERR_CAP];
    auto ensure = [&](pfhip_buffer*& buf, size_t bytes) {
      if (!buf || buf->size < bytes) {
        pfhip_release_buffer(m->b, buf);
        buf = pfhip_create_empty_buffer(m->b, bytes, e2, sizeof e2);
        PF_CHECK(buf, e2);
      }
    };
    ensure(m->ids_buf, M * 4);
    ensure(m->logits_buf, M * m->cfg.classes * 4);
    PF_CHECK(pfhip_write_buffer(m->b, m->ids_buf, 0, ids, M * 4, e2, sizeof e2) == 0, e2);
    // wasm.ts:753-764: an all-ones mask is elided
    bool use_mask = false;
    if (mask)
      for (size_t i = 0; i < M; ++i)
        if (mask[i] != 1) {
          use_mask = true;
          break;
        }
    if (use_mask) {
      ensure(m->mask_buf, M);
      PF_CHECK(pfhip_write_buffer(m->b, m->mask_buf, 0, mask, M, e2, sizeof e2) == 0, e2);
    }
    PF_CHECK(pfhip_model_forward_device(m, m->ids_buf, use_mask ? m->mask_buf : nullptr, batch, seq_len,
                                        m->logits_buf, e2, sizeof e2) == 0,
             e2);
    PF_CHECK(pfhip_read_buffer(m->b, m->logits_buf, 0, logits, M * m->cfg.classes * 4, e2, sizeof e2) == 0, e2);
    return 0;
  } catch (const std::exception& ex) {
    set_err(err, cap, ex.what());
    return -1;
  }
}

int pfhip_model_read_tap(pfhip_model* m, const char* name, void* dst, size_t n, char* err, size_t cap) {
  try {
    PF_CHECK(m && name && dst, "null argument");
    auto it = m->tap.find(name);
    PF_CHECK(it != m->tap.end(), std::string("no tap \"") + name + "\" (enable taps before the forward)");
    PF_CHECK(n <= it->second.size(), "tap read larger than the tap");
    memcpy(dst, it->second.data(), n);
    return 0;
  } catch (const std::exception& ex) {
    set_err(err, cap, ex.what());
    return -1;
  }
}

int pfhip_rope_tables(const pfhip_model_config* cfg, uint32_t T, uint16_t* cos_t, uint16_t* sin_t) {
  if (!cfg || !cos_t || !sin_t) return -1;
  std::vector<uint16_t> cs, sn;
  build_rope_tables(*cfg, (int)T, cs, sn);
  memcpy(cos_t, cs.data(), cs.size() * 2);
  memcpy(sin_t, sn.data(), sn.size() * 2);
  return 0;
}

}  // extern "C"
