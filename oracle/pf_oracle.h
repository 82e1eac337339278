/*
 * pf_oracle.h — CPU restatement of textsift's WASM forward path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * backend and the CPU baseline timed beside it. Only tests/, the smoke check
 * in __graft_entry__.py and bench.py's cpu_baseline leg may load it; the
 * product library (textsift_amd) never links, loads or calls it.
 *
 * Every function restates one function of the reference, cited as
 * packages/textsift/src/<file>:<line>. Numerics follow the WASM build:
 *   - fp16 widen is the non-IEEE bit trick of zig/math.zig:45-52,
 *   - f32->fp16 is RNE for normals, round-half-up for subnormals
 *     (zig/math.zig:54-82),
 *   - every relaxed_madd site (c/fma.c:10-13) is a fused fmaf (V8 on x86-64
 *     fuses), every other multiply/add is rounded separately (built with
 *     -ffp-contract=off).
 * Zig's std @exp is stood in for by the C library's expf; that last-ulp
 * choice is not pinned by any reference test ("parity unpinned" for
 * softmax_f32's exp, the scalar sigmoid and the scalar attention tail).
 */
#ifndef PF_ORACLE_H
#define PF_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- conversions: zig/math.zig ---- */
float pfo_fp16_to_f32(uint16_t h);          /* :45-52  (non-IEEE subnormals) */
uint16_t pfo_f32_to_fp16(float f);          /* :54-82 */
void pfo_fp16_to_f32_n(const uint16_t* src, float* dst, size_t n);
void pfo_f32_to_fp16_n(const float* src, uint16_t* dst, size_t n);
float pfo_exp_approx(float x);              /* wasm_exports.zig:812-838 (one lane) */

/* ---- kernels: zig/wasm_exports.zig ---- */
void pfo_rms_norm(const uint16_t* x, const uint16_t* gamma, uint16_t* out,
                  uint32_t T, uint32_t D, float eps);                       /* :186-218 */
void pfo_rms_norm_fp16_to_f32(const uint16_t* x, const uint16_t* gamma, float* out,
                              uint32_t T, uint32_t D, float eps);           /* :220-270 */
void pfo_add_rmsnorm_fp16_to_f32(const uint16_t* a, const uint16_t* b, const uint16_t* gamma,
                                 uint16_t* sum_out, float* norm_out,
                                 uint32_t T, uint32_t D, float eps);        /* :288-350 */
void pfo_topk_partial_f32(const float* x, int32_t* out_idx, float* out_val,
                          uint32_t rows, uint32_t cols, uint32_t k);        /* :367-426 */
/* x_f32 / out_f32 select the four exports of :713-766 */
void pfo_matmul_int4block(int x_f32, int out_f32, const void* x, const uint8_t* w_int4,
                          const uint16_t* w_scales, const uint8_t* w_zp /* may be NULL */,
                          const uint16_t* bias, void* out,
                          uint32_t T, uint32_t N, uint32_t D);              /* :560-707 */
void pfo_swiglu_clamp_f32(const float* gate_up, float* out, uint32_t T, uint32_t D); /* :855-903 */
void pfo_softmax_f32(const float* x, float* out, uint32_t rows, uint32_t cols);     /* :919-958 */
void pfo_add_fp16(const uint16_t* a, const uint16_t* b, uint16_t* out, uint32_t n); /* :969-990 */
void pfo_gather_f32(const float* src, const int32_t* idx, float* dst, uint32_t m, uint32_t D); /* :1127-1143 */
void pfo_scatter_add_weighted_f32(float* target, const float* values, const int32_t* idx,
                                  const float* weights, uint32_t m, uint32_t D); /* :1027-1055 */
void pfo_cast_f32_to_fp16_scaled(const float* src, uint16_t* dst, uint32_t n, float scale); /* :1153-1164 */
void pfo_banded_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                          const float* sinks, const uint8_t* mask /* may be NULL */,
                          uint16_t* out, uint32_t T, uint32_t Hq, uint32_t Hkv,
                          uint32_t head_dim, uint32_t window,
                          uint32_t h_q_start, uint32_t h_q_end);
/* IEEE f32 -> fp16 (round to nearest even, subnormals kept): WGSL f16(). */
void pfo_f2h_ieee(const float* x, uint16_t* out, size_t n);
/* banded_attention.wgsl (the reference's GPU path): libm exp, the shader's
 * reduction orders, IEEE fp16 conversions. */
void pfo_banded_attention_wgsl(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* sinks,
                               const uint8_t* mask, uint16_t* out, uint32_t T, uint32_t Hq, uint32_t Hkv,
                               uint32_t Dh, uint32_t W);             /* :1286-1432 */
void pfo_rope_apply(uint16_t* qk, const uint16_t* cos_t, const uint16_t* sin_t,
                    uint32_t T, uint32_t H, uint32_t head_dim);              /* :1460-1502 */
void pfo_embed_lookup_int4(const uint8_t* embed_int4, const uint16_t* embed_scales,
                           const uint8_t* embed_zp, const int32_t* ids, uint16_t* out,
                           uint32_t T, uint32_t V, uint32_t D);              /* :1523-1573 */

/* ---- host-side pieces of the forward (browser/inference/ TS files) ---- */
typedef struct {
  uint32_t hidden, heads, kv_heads, head_dim, window, dff, experts, topk, classes, vocab, layers;
  float eps;
  double rope_theta, rope_factor, rope_beta_fast, rope_beta_slow;
  uint32_t rope_orig_max, rope_truncate;
} pfo_config;

/* rope.ts:27-144 (computeYarnInvFreq, getYarnAttentionScaling, computeRopeTables) */
void pfo_rope_tables(const pfo_config* cfg, uint32_t T, uint16_t* cos_t, uint16_t* sin_t);

typedef struct {
  const uint8_t* int4;
  const uint16_t* scales;
  const uint8_t* zp;       /* may be NULL (symmetric decode) */
  const uint16_t* bias;
} pfo_qweight;

typedef struct {
  const uint16_t* input_ln;
  const uint16_t* post_ln;
  pfo_qweight q, k, v, o;
  const float* sinks;
  pfo_qweight router;      /* int4 router, model path (block.ts:49-102) */
  pfo_qweight gate_up;     /* [E, 2*dff, D/2] ... (expert.ts:1-53) */
  pfo_qweight down;        /* [E, D, dff/2] ... */
} pfo_layer;

typedef struct {
  const uint8_t* embed_int4;
  const uint16_t* embed_scales;
  const uint8_t* embed_zp;
  const pfo_layer* layers;
  const uint16_t* final_ln;
  pfo_qweight score;
} pfo_model;

/* Router on f32 logits (block.ts:96-101): top-k, softmax over k, x(1/k). */
void pfo_router_select(const float* logits, int32_t* idx, float* weights,
                       uint32_t T, uint32_t E, uint32_t K);

/* Expert-major MoE dispatch (expert.ts:104-212). n_slices = 1 restates the
 * single-thread loop; n_slices > 1 restates the worker-pool token slicing
 * of mt-expert.ts:63-191 (same numerics per slice, run on n_slices threads). */
int pfo_expert_dispatch(const pfo_config* cfg, const pfo_layer* layer, const float* hidden_f32,
                        const int32_t* routing_idx, const float* routing_w,
                        uint16_t* out, uint32_t T, int n_slices);

/* modelForward (model.ts:50-105) -> fp16 logits [T, classes].
 * n_threads = 1 is WasmBackend's single-thread path; n_threads > 1 uses the
 * MtPool partitioning (T-slices for GEMMs/norms, H_q slices for attention,
 * token slices for the MoE) and runs it on that many threads. mask may be
 * NULL (all ones; wasm.ts:753-764). Returns 0 on success. */
int pfo_model_forward(const pfo_config* cfg, const pfo_model* m, const int32_t* ids,
                      const uint8_t* mask, uint32_t T, int n_threads, uint16_t* logits);

/* One transformer block (block.ts:108-197); in/out fp16 [T, hidden]. */
/* pfo_model_forward that also returns every layer's routed expert ids
 * (ridx_out [layers][T][topk], NULL to skip). */
int pfo_model_forward_route(const pfo_config* cfg, const pfo_model* m, const int32_t* ids,
                            const uint8_t* mask, uint32_t T, int n_threads, uint16_t* logits,
                            int32_t* ridx_out);
int pfo_block_forward(const pfo_config* cfg, const pfo_layer* layer, const uint16_t* input,
                      uint16_t* output, const uint16_t* cos_t, const uint16_t* sin_t,
                      const uint8_t* mask, uint32_t T, int n_threads);

#ifdef __cplusplus
}
#endif
#endif
