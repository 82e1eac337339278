// pfhip_internal.h — host-side structures shared by the runtime, the kernel
// launchers and the forward orchestration.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/pfhip.h"

struct pfhip_buffer {
  void* ptr = nullptr;
  size_t size = 0;
  pfhip_backend* owner = nullptr;
};

namespace pf {

struct Error : std::runtime_error {
  explicit Error(const std::string& m) : std::runtime_error(m) {}
};

#define PF_HIP(expr)                                                                              \
  do {                                                                                            \
    hipError_t e_ = (expr);                                                                       \
    if (e_ != hipSuccess)                                                                         \
      throw ::pf::Error(std::string(#expr) + " failed: " + hipGetErrorString(e_) + " (" __FILE__ \
                        ":" + std::to_string(__LINE__) + ")");                                    \
  } while (0)

#define PF_CHECK(cond, msg)                       \
  do {                                            \
    if (!(cond)) throw ::pf::Error(std::string(msg)); \
  } while (0)

struct ProfPending {
  const char* name;
  hipEvent_t start, stop;
};

}  // namespace pf

struct pfhip_backend {
  int device = 0;
  int num_cus = 256;  // compute units of the device
  hipStream_t stream = nullptr;
  std::string device_name;
  bool encoder_open = false;
  // profiling
  bool profiling = false;
  std::string profile_only;  // record only launches of this name ("" = all)
  std::vector<pf::ProfPending> pending;
  std::vector<hipEvent_t> event_pool;
  std::map<std::string, std::pair<long, double>> prof;  // name -> (launches, total ms)
  std::string report;
};

struct pfhip_encoder {
  pfhip_backend* b = nullptr;
  int dispatches = 0;
};

namespace pf {

// Brackets one kernel launch with events when profiling is on.
struct ProfScope {
  pfhip_backend* b;
  const char* name;
  hipEvent_t start = nullptr, stop = nullptr;
  ProfScope(pfhip_backend* b_, const char* n);
  ~ProfScope() noexcept(false);
};

void prof_flush(pfhip_backend* b);  // synchronises and accumulates pending events
// Raises kern's dynamic LDS limit to at least `bytes` on the current device
// (once per kernel and device; thread-safe). Call before launching with
// more than 64 KB of dynamic LDS.
void allow_lds(const void* kern, size_t bytes);

void set_err(char* err, size_t cap, const std::string& msg);

// ---------------------------------------------------------------- kernels
// Launchers live in the .hip translation units; every one launches on
// b->stream, validates its shapes on the host first and throws pf::Error.

// MatMulNBits int4 GEMM.
// F16: activations are one fp16 plane. SPLIT: f32 activations carried as two
// fp16 planes, hi = fp16(v) and lo = fp16(v - hi) (22 significant bits), which
// enter the MFMA as two products per block into the same partial sum.
enum class XKind { F16, SPLIT };
// F32_TOPK (gemm_w4, N == 128, one column tile): F32, then the router
// top-4 + softmax of each output row into topk_idx / topk_w.
enum class Epi { F16, F32, ROPE_F16, SWIGLU_SPLIT, SWIGLU_F16, F32_TOPK };

struct GemmArgs {
  const void* x = nullptr;       // activations [rows][K] fp16 (the hi plane in SPLIT mode)
  const uint16_t* x_lo = nullptr;  // SPLIT: the lo plane, same row stride
  int ldx = 0;                   // row stride in elements
  const int32_t* row_map = nullptr;  // optional gather: logical row r reads x row row_map[r]
  const uint8_t* w = nullptr;    // [N][K/2] uint4 (per group stride w_gs bytes)
  const uint16_t* ws = nullptr;  // [N][K/32] fp16 scales
  const uint8_t* wz = nullptr;   // [N][ceil(K/64)] packed uint4 zero-points, NULL = 0
  const uint16_t* bias = nullptr;  // [N] fp16, NULL = 0
  size_t w_gs = 0, ws_gs = 0, wz_gs = 0, bias_gs = 0;  // per-expert strides (elements)
  // gemm_w4 only: repacked weights in w, and per block (fp16 -(1024+zp), fp16 scale)
  const uint32_t* wsz = nullptr;  // [N][K/32]
  size_t wsz_gs = 0;
  // gemm_w4, router top-k tile only: fp16 weights [N][K] instead of w / wsz
  const uint16_t* w16 = nullptr;
  void* out = nullptr;
  uint16_t* out_lo = nullptr;    // SWIGLU_SPLIT: lo plane of the output
  // F16 epilogue with direct stores: the fp16-rounded outputs also widened
  // to f32 here ([M][ldo], IEEE widening, exact), out may then be NULL (the
  // classifier's logits without a separate cast)
  float* out_f32w = nullptr;
  int ldo = 0;
  int M = 0, N = 0, K = 0;
  // grouped (per-expert) mode
  const int32_t* tiles = nullptr;      // [max_tiles][4] = (expert, row0, rows, 0)
  const int32_t* num_tiles = nullptr;  // device scalar
  int max_tiles = 0;
  // RoPE epilogue
  const float* rope_cos = nullptr;  // [seq_len][head_dim/2]: fp16 table entries widened as
  const float* rope_sin = nullptr;  // wasm_h2f widens them (zig/math.zig:45-52)
  const uint16_t* rope_pairs = nullptr;  // [seq_len][head_dim/2][cos, sin] fp16 bits (gemm_w4)
  int seq_len = 0;
  int rope_cols = 0;                   // columns [0, rope_cols) are rotated
  // F32_TOPK epilogue: [M][topk_k] expert ids and routing weights (times topk_wscale)
  int32_t* topk_idx = nullptr;
  float* topk_w = nullptr;
  int topk_k = 0;
  float topk_wscale = 1.0f;
  // F32_TOPK: when set, [M / BT][128] counts of each tile's rows routed to each expert
  int32_t* topk_counts = nullptr;
  // F32_TOPK on a single 16-row tile (M <= 16): when plan_slot_of is set, the
  // same workgroup then builds the routing plan of its rows (the outputs of
  // moe_route: expert_off [E + 1], slot_token, slot_of, the expert tile list
  // of plan_tile_t-row tiles and num_tiles), one launch fewer per layer
  int32_t* plan_expert_off = nullptr;
  int32_t* plan_slot_token = nullptr;
  int32_t* plan_slot_of = nullptr;
  int32_t* plan_tiles = nullptr;
  int32_t* plan_num_tiles = nullptr;
  int plan_tile_t = 0;
  // Residual add + RMSNorm on the way in (gemm_w4, 16-token tile, K == 640):
  // x is the fp16 O projection output o; the kernel forms h2 = fp16(o + res)
  // and xn = fp16(h2 * inv_rms(o + res) * gamma), writes both, and multiplies xn.
  const uint16_t* nrm_res = nullptr;
  const uint16_t* nrm_gamma = nullptr;
  uint16_t* nrm_h = nullptr;
  uint16_t* nrm_xn = nullptr;
  float nrm_eps = 0.0f;
  // gemm_w4: stage the output tile through LDS and store whole 16-byte units
  // (set by gemm_w4 itself when the output layout allows it)
  int out_staged = 0;
};

void gemm_int4(pfhip_backend* b, const GemmArgs& a, XKind xk, Epi epi, bool grouped, int tile_t,
               const char* prof_name);

// Tile of the grouped expert GEMMs for M tokens routed to topk of experts:
// t tokens per tile (128, 64 or 16; also the routing plan's tile) and wf
// 16-row weight fragments per wave (gemm_w4). The forward and the moe_ffn
// named kernel choose it the same way.
struct ExpertTile {
  int t, wf;
};
ExpertTile expert_tile(int M, int topk, int experts, bool fp16, int D, int F);

// Scale-folded int4 GEMM (gemm_w4.hip): weights prepared by w4_prepare;
// K % 128 == 0. tile_t x wf selects the tile (BT tokens x 64*wf rows):
// (128, 4), (128, 2), (64, 5), (64, 1), and the small-M tiles (16, 1) and
// (16, 2) that load all of K (640 or 896) at once.
void gemm_w4(pfhip_backend* b, const GemmArgs& a, XKind xk, Epi epi, bool grouped, int tile_t, int wf,
             const char* prof_name);
// O projection (gemm_w4 weights, N == 640, bias folded as in gemm_w4) with the
// residual add and RMSNorm fused: h_out = fp16(fp16(x.w + bias) + resid),
// xn_out = fp16(h_out * inv_rms * gamma) (fp16 numerics).
void gemm_w4_add_rmsnorm(pfhip_backend* b, const GemmArgs& a, const uint16_t* resid, const uint16_t* gamma,
                         uint16_t* h_out, uint16_t* xn_out, float eps);
// MatMulNBits weight [rows][K/2] + scales + zero-points -> the gemm_w4 form:
// w_out [rows][K/8] repacked dwords, sz_out [rows][K/32] (offset, scale) pairs.
void w4_prepare(pfhip_backend* b, const uint8_t* w, const uint16_t* ws, const uint8_t* wz, uint32_t* w_out,
                uint32_t* sz_out, int rows, int K);

// GatherBlockQuantized embedding: out fp16 [T][D]. stream_out: non-temporal
// stores (the output is not read by the next kernel: the stand-alone op);
// the forward keeps them cached for the RMSNorm that reads them next.
void embed_lookup(pfhip_backend* b, const uint8_t* q, const uint16_t* s, const uint8_t* zp, const int32_t* ids,
                  uint16_t* out, int T, int V, int D, bool stream_out = false);

// embed_lookup into h, then rms_norm_f16 of h into out: one kernel for the
// model's width (D = 640, aligned operands), bit-identical to the two.
void embed_rms_norm_f16(pfhip_backend* b, const uint8_t* q, const uint16_t* s, const uint8_t* zp, const int32_t* ids,
                        const uint16_t* g, uint16_t* h, uint16_t* out, int T, int V, int D, float eps);

// RMSNorm family. The *_split variants write the f32 result as hi/lo fp16
// planes (norm_hi, norm_lo) for SPLIT GEMM inputs.
void rms_norm_f16(pfhip_backend* b, const uint16_t* x, const uint16_t* g, uint16_t* out, int T, int D, float eps);
void rms_norm_f32(pfhip_backend* b, const uint16_t* x, const uint16_t* g, float* out, int T, int D, float eps);
void rms_norm_split(pfhip_backend* b, const uint16_t* x, const uint16_t* g, uint16_t* hi, uint16_t* lo, int T, int D,
                    float eps);
void add_rms_norm_f32(pfhip_backend* b, const uint16_t* a, const uint16_t* bb, const uint16_t* g, uint16_t* sum_out,
                      float* norm_out, int T, int D, float eps);
void add_rms_norm_f16(pfhip_backend* b, const uint16_t* a, const uint16_t* bb, const uint16_t* g, uint16_t* sum_out,
                      uint16_t* norm_out, int T, int D, float eps);
void add_rms_norm_split(pfhip_backend* b, const uint16_t* a, const uint16_t* bb, const uint16_t* g,
                        uint16_t* sum_out, uint16_t* hi, uint16_t* lo, int T, int D, float eps);
// f32 -> (hi, lo) fp16 planes.
void split_f32(pfhip_backend* b, const float* x, uint16_t* hi, uint16_t* lo, size_t n);

// Element-wise.
void add_f16(pfhip_backend* b, const uint16_t* a, const uint16_t* bb, uint16_t* out, size_t n);
void cast_f16_f32(pfhip_backend* b, const uint16_t* src, float* dst, size_t n);
void cast_f32_f16_scaled(pfhip_backend* b, const float* src, uint16_t* dst, size_t n, float scale);
void zero_f32(pfhip_backend* b, float* p, size_t n);
void swiglu_f32(pfhip_backend* b, const float* gu, float* out, int rows, int dff);
void rope_apply(pfhip_backend* b, uint16_t* qk, const uint16_t* c, const uint16_t* s, int T, int H, int hd,
                int row_stride, int seq_len);

// Routing.
void router_topk(pfhip_backend* b, const float* logits, int32_t* idx, float* w, int T, int E, int K,
                 float weight_scale);
struct MoePlan {
  int32_t* counts;      // [nblk][E]
  int32_t* blk_off;     // [nblk][E]
  int32_t* expert_off;  // [E+1]
  int32_t* slot_token;  // [T*K]  token of each expert-sorted slot
  int32_t* slot_of;     // [T*K]  slot of (token, k)
  int32_t* tiles;       // [max_tiles][4]
  int32_t* num_tiles;   // [1]
  int32_t* tile_counts; // [ceil(T / 16)][E] expert counts per router tile (moe_route_counts)
  int max_tiles;
  int tile_t;
};
int moe_max_tiles(int T, int K, int E, int tile_t);
size_t moe_plan_bytes(int T, int K, int E, int tile_t);
MoePlan moe_plan_carve(void* base, int T, int K, int E, int tile_t);
void moe_route(pfhip_backend* b, const int32_t* idx, int T, int K, int E, const MoePlan& plan);
// The same plan from counts[tile][e] of the tokens' tiles of tile_rows rows
// (tile_rows divides 1024; written by the router GEMM's top-k epilogue):
// one kernel instead of three.
void moe_route_counts(pfhip_backend* b, const int32_t* idx, const int32_t* counts, int tile_rows, int T, int K, int E,
                      const MoePlan& plan);
// y: the expert outputs in slot order, fp16 when y16 (the fp16 numerics), else f32;
// residual NULL: no residual (the outputs hold the MoE result alone).
void moe_combine(pfhip_backend* b, const int32_t* idx, const float* w, const int32_t* slot_of, const void* y,
                 bool y16, const uint16_t* residual, uint16_t* moe_out, uint16_t* h_out, int T, int K, int D);
// norm_lo == NULL: the norm output is one fp16 plane in norm_hi.
void moe_combine_norm(pfhip_backend* b, const int32_t* idx, const float* w, const int32_t* slot_of, const void* y,
                      bool y16, const uint16_t* residual, uint16_t* h_out, const uint16_t* gamma, uint16_t* norm_hi,
                      uint16_t* norm_lo, int T, int K, int D, float eps);
// fp16-weight router GEMM (MFMA); wt: scratch for W^T, E * D fp16, 16-byte aligned.
// [rows][cols] fp16 -> [cols][rows]
void transpose_f16(pfhip_backend* b, const uint16_t* src, uint16_t* dst, int rows, int cols);
void router_f16w(pfhip_backend* b, const uint16_t* x, const uint16_t* w, const uint16_t* bias, float* logits, int T,
                 int D, int E, uint16_t* wt);

// Banded GQA attention with sinks.
struct AttnArgs {
  const uint16_t* q; int q_stride;
  const uint16_t* k; int k_stride;
  const uint16_t* v; int v_stride;
  const float* sinks;   // [Hq] or NULL (no sink = -inf)
  const uint8_t* mask;  // [B*T] or NULL
  uint16_t* out; int out_stride;
  int B, T, Hq, Hkv, head_dim, window;
  float scale;
  int hw_exp;           // 1: hardware exp2 softmax (the GPU paths' numerics); 0: the WASM path's
  int head_groups = 1;  // set by the launcher: workgroups per KV head (an even split of its Hq/Hkv query heads)
};
void banded_attention(pfhip_backend* b, const AttnArgs& a);

// Reference-layout kernels kept for the named-dispatch surface.
void qmoe_gate_up_ref(pfhip_backend* b, const float* x, const int32_t* ridx, const uint8_t* w, const uint16_t* ws,
                      const uint8_t* wz, const uint16_t* bias, float* out, int T, int K, int N, int D);
void qmoe_down_scatter_ref(pfhip_backend* b, const float* glu, const int32_t* ridx, const float* rw,
                           const uint8_t* w, const uint16_t* ws, const uint8_t* wz, const uint16_t* bias, float* acc,
                           int T, int K, int N, int D);

// Fixed device scratch of the allocation-free forward entry (noalloc.hip):
// PFHIP_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends. Returns
// its address on `device` (looked up once per device, with that device current).
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)PFHIP_NOALLOC_SCRATCH_MIB << 20;
void* noalloc_scratch(int device);

// Plain device copy of `bytes` (multiple of 16, 16-byte aligned), and the
// calibration workloads of known size for the HBM counters: the same copy
// with HBM -> LDS loads, and a gather of n 16-byte units at idx[i] % table_units.
void copy16(pfhip_backend* b, const void* src, void* dst, size_t bytes);
void copy16_lds(pfhip_backend* b, const void* src, void* dst, size_t bytes);
void gather16(pfhip_backend* b, const void* table, uint32_t table_units, const int32_t* idx, void* dst, size_t n);

// Exhaustive checks of the fast math helpers (tests only): which = 0 checks
// div_one_plus against IEEE division, 1 checks exp_approx_fast against
// exp_approx. out: [mismatches, first mismatching bit pattern, outside-domain].
void probe_fast_math(pfhip_backend* b, int which, uint32_t lo, uint32_t hi, uint32_t* out);

// Layout probe for the MFMA operand assumption (tests only).
void probe_mfma_f16(pfhip_backend* b, const uint16_t* a, const uint16_t* bm, float* d);

}  // namespace pf
