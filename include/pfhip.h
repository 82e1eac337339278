/*
 * pfhip.h — C ABI of the MI355X (gfx950) backend for textsift's
 * privacy-filter forward pass.
 *
 * The reference's native GPU backend reaches the GPU through an N-API module
 * whose surface is listed in packages/textsift/src/native/backend.ts:34-60
 * (NativeApi) and implemented per platform in native/napi.zig:546-864 over
 * the C bridge native/vulkan/bridge.h:33-97. This header is the same surface
 * for HIP: plain pointers and sizes, opaque handles, no torch types.
 *
 * Errors: functions return 0 (or a non-NULL handle) on success. On failure
 * they return a negative status (or NULL) and, when err != NULL, write a
 * NUL-terminated message into err[0..err_cap) (bridge.h:5-8,41-44 use the
 * same caller-provided buffer convention). No function aborts the process.
 *
 * Threading: one backend is used from one host thread at a time
 * (privacy-filter.ts:523-527 serialises calls). All work of a backend runs on
 * its own HIP stream.
 */
#ifndef PFHIP_H
#define PFHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct pfhip_backend pfhip_backend;
typedef struct pfhip_buffer pfhip_buffer;
typedef struct pfhip_encoder pfhip_encoder;
typedef struct pfhip_model pfhip_model;

#define PFHIP_ERR_CAP 1024

/* ------------------------------------------------------------------------
 * Lifecycle — replaces ts_vk_create_backend / ts_vk_destroy_backend /
 * ts_vk_device_name (native/vulkan/bridge.h:41-52; napi.zig:561-600).
 * device: HIP device ordinal. Fails (NULL) if the device is not gfx950.
 * --------------------------------------------------------------------- */
pfhip_backend* pfhip_create_backend(int device, char* err, size_t err_cap);
void pfhip_destroy_backend(pfhip_backend* b);
int pfhip_device_name(pfhip_backend* b, char* out, size_t cap);

/* ------------------------------------------------------------------------
 * Buffers — replaces ts_vk_create_buffer / create_empty / release / write /
 * read (bridge.h:62-80; napi.zig:603-697). Device memory (hipMalloc).
 * create_buffer copies `n` bytes from host; create_empty zero-fills.
 * --------------------------------------------------------------------- */
pfhip_buffer* pfhip_create_buffer(pfhip_backend* b, const void* bytes, size_t n, char* err, size_t err_cap);
pfhip_buffer* pfhip_create_empty_buffer(pfhip_backend* b, size_t n, char* err, size_t err_cap);
void pfhip_release_buffer(pfhip_backend* b, pfhip_buffer* buf);
int pfhip_write_buffer(pfhip_backend* b, pfhip_buffer* buf, size_t offset, const void* bytes, size_t n, char* err,
                       size_t err_cap);
int pfhip_read_buffer(pfhip_backend* b, pfhip_buffer* buf, size_t offset, void* out, size_t n, char* err,
                      size_t err_cap);
size_t pfhip_buffer_size(const pfhip_buffer* buf);
/* Device address of a buffer (for callers that pass it to their own HIP code). */
void* pfhip_buffer_device_ptr(const pfhip_buffer* buf);

/* ------------------------------------------------------------------------
 * Kernel dispatch by name — replaces vulkanDispatchOneShot /
 * BeginEncoder / EnqueueDispatch / SubmitAndReadback
 * (napi.zig:741-862; bridge.h:84-97).
 *
 * bindings: the kernel's buffers in the reference's binding order;
 * push: the kernel's uniform block (the reference's `Dims` struct bytes);
 * grid: accepted for interface parity and ignored — each HIP kernel derives
 * its launch geometry from `push` (workgroups here are not 64-thread WGSL
 * workgroups). pfhip_kernel_names() lists every registered kernel as one
 * "name bindings push_bytes" line; the reference's 15 names
 * (vulkan_backend.zig:51-112) keep their binding order and Dims layout so
 * its conformance fixtures run unchanged.
 *
 * An encoder records dispatches on the backend's stream; submit waits for
 * them, copies `n` bytes of `out` at `offset` into `dst` and releases the
 * encoder (napi.zig:833-862). Only one encoder may be open per backend.
 * --------------------------------------------------------------------- */
int pfhip_dispatch_one_shot(pfhip_backend* b, const char* name, pfhip_buffer* const* bindings, uint32_t n_bindings,
                            const void* push, size_t push_len, const uint32_t grid[3], char* err, size_t err_cap);
pfhip_encoder* pfhip_begin_encoder(pfhip_backend* b, char* err, size_t err_cap);
int pfhip_enqueue_dispatch(pfhip_encoder* e, const char* name, pfhip_buffer* const* bindings, uint32_t n_bindings,
                           const void* push, size_t push_len, const uint32_t grid[3], char* err, size_t err_cap);
int pfhip_submit_and_readback(pfhip_encoder* e, pfhip_buffer* out, size_t offset, void* dst, size_t n, char* err,
                              size_t err_cap);
void pfhip_discard_encoder(pfhip_encoder* e);
/* Newline-separated "name bindings push_bytes" lines for every registered kernel. */
const char* pfhip_kernel_names(void);

/* ------------------------------------------------------------------------
 * Whole forward — the 148-dispatch sequence of NodeBackend.forward
 * (native/backend.ts:433-704) as one call over B sequences of T tokens.
 *
 * Weights are set by the names NodeBackend.uploadWeights gives them
 * (native/backend.ts:140-236: "embed.int4", "layers.0.attn.q_proj.scales",
 * "layers.0.experts.gate_up.zp", "final_norm", "score.bias", ...), with the
 * ONNX byte layouts (MatMulNBits / GatherBlockQuantized; router scales and
 * bias already fp16, expert zero-points materialised as 0x88).
 * finalize() checks every tensor is present with the right size and
 * repacks what the kernels want repacked.
 * --------------------------------------------------------------------- */
typedef struct {
  uint32_t hidden;        /* 640 */
  uint32_t heads;         /* 14  */
  uint32_t kv_heads;      /* 2   */
  uint32_t head_dim;      /* 64  */
  uint32_t window;        /* 128 */
  uint32_t dff;           /* 640 */
  uint32_t experts;       /* 128 */
  uint32_t topk;          /* 4   */
  uint32_t classes;       /* 33  */
  uint32_t vocab;         /* 200064 */
  uint32_t layers;        /* 8   */
  float eps;              /* 1e-5 */
  double rope_theta;      /* 150000 */
  double rope_factor;     /* 32 */
  double rope_beta_fast;  /* 32 */
  double rope_beta_slow;  /* 1 */
  uint32_t rope_orig_max; /* 4096 */
  uint32_t rope_truncate; /* 0 */
  /* Numerics of the GEMM inputs:
   * PFHIP_PRECISION_FP16  activations enter the int4 GEMMs as fp16 and the
   *                       block scale is folded into fp16 weights (what the
   *                       reference's GPU paths feed their GEMMs);
   * PFHIP_PRECISION_SPLIT activations keep f32 precision as hi/lo fp16 planes
   *                       and weights enter as exact (q - zp) with the scale
   *                       applied per block in f32 (the WASM path's numerics). */
  uint32_t precision;
} pfhip_model_config;

#define PFHIP_PRECISION_FP16 0u
#define PFHIP_PRECISION_SPLIT 1u

pfhip_model* pfhip_model_create(pfhip_backend* b, const pfhip_model_config* cfg, char* err, size_t err_cap);
void pfhip_model_destroy(pfhip_model* m);
int pfhip_model_set_weight(pfhip_model* m, const char* name, const void* bytes, size_t n, char* err, size_t err_cap);
int pfhip_model_finalize(pfhip_model* m, char* err, size_t err_cap);

/* Host in / host out (WasmBackend.forward contract, browser/backends/wasm.ts:728-805):
 * ids int32 [batch*seq_len], mask uint8 [batch*seq_len] or NULL (all ones),
 * logits float32 [batch*seq_len*classes] = fp16-rounded logits widened. */
int pfhip_model_forward(pfhip_model* m, const int32_t* ids, const uint8_t* mask, uint32_t batch, uint32_t seq_len,
                        float* logits, char* err, size_t err_cap);
/* Device in / device out: same, with inputs already resident in HBM.
 * mask may be NULL. Returns after the forward has completed. */
int pfhip_model_forward_device(pfhip_model* m, pfhip_buffer* ids, pfhip_buffer* mask, uint32_t batch,
                               uint32_t seq_len, pfhip_buffer* logits, char* err, size_t err_cap);
/* Allocation-free variant of pfhip_model_forward_device. It has no
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments, kernels and results as
 * pfhip_model_forward_device, but the forward's scratch (activations, routing
 * plan) is a fixed device array of PFHIP_NOALLOC_SCRATCH_MIB MiB per GPU,
 * held from the library's set-up on that GPU (pfhip_create_backend) until the
 * process ends, and nothing is allocated: batch * seq_len must fit that array
 * (one 2048-token sequence of the privacy-filter model does) and seq_len must
 * not exceed the RoPE tables already built (pfhip_model_finalize builds them
 * for 2048 positions; a longer pfhip_model_forward_device call grows them).
 * Larger requests fail with an error before any work. Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (from several
 * threads, backends or models) race. Debug taps are not recorded. */
#define PFHIP_NOALLOC_SCRATCH_MIB 80
int pfhip_model_forward_device_noalloc(pfhip_model* m, pfhip_buffer* ids, pfhip_buffer* mask, uint32_t batch,
                                       uint32_t seq_len, pfhip_buffer* logits, char* err, size_t err_cap);
/* Debug taps of the last forward (for parity tests): copies a named
 * intermediate ("h.L" residual after layer L, "logits16") to the host. */
int pfhip_model_read_tap(pfhip_model* m, const char* name, void* dst, size_t n, char* err, size_t err_cap);
/* Taps are recorded only while enabled (they copy every intermediate to the
 * host). Names: "qkv.L", "att.L", "h2.L", "router.L", "ridx.L", "rw.L",
 * "h.L" for layer L, and "logits16". */
int pfhip_model_enable_taps(pfhip_model* m, int on);
/* HIP graphs for pfhip_model_forward_device / pfhip_model_forward (on by
 * default). The reference records a forward's whole dispatch sequence into
 * one command encoder and submits it once (native/backend.ts:485,693); here
 * the first call for a (batch, seq_len, ids, mask, logits) combination runs
 * eagerly, the second captures its launches into a HIP graph and every later
 * one replays it (16 combinations are kept, the oldest dropped first). Buffer
 * contents may change between calls; the buffers themselves are part of the
 * key. Forwards with taps or profiling enabled always run eagerly, and the
 * graphs are dropped whenever weights are set, the model is finalized, or the
 * scratch or RoPE tables grow. on = 0 drops them and runs eagerly. */
int pfhip_model_enable_graphs(pfhip_model* m, int on);

/* The YARN RoPE tables the forward uses for sequence length T
 * (browser/inference/rope.ts:27-144): fp16 bits [T][head_dim/2] each. */
int pfhip_rope_tables(const pfhip_model_config* cfg, uint32_t T, uint16_t* cos_t, uint16_t* sin_t);

/* ------------------------------------------------------------------------
 * Profiling: when enabled, every kernel launch of the backend is bracketed by
 * HIP events on the backend's stream and its duration accumulated per kernel
 * name. report() writes "name launches total_ms" lines.
 * --------------------------------------------------------------------- */
int pfhip_profile_enable(pfhip_backend* b, int on);
/* Restricts recording to launches named `name` (NULL or "" = every launch),
 * so a timed region can bracket one kernel without timing all of them. */
int pfhip_profile_select(pfhip_backend* b, const char* name);
int pfhip_profile_reset(pfhip_backend* b);
int pfhip_profile_report(pfhip_backend* b, char* out, size_t cap);

/* ------------------------------------------------------------------------
 * Host-side span decoding of the forward's logits.
 *
 * ViterbiDecoder.decode (packages/textsift/src/browser/inference/viterbi.ts:
 * 85-146, tables :159-219): the most likely BIOES tag sequence of each of
 * `batch` sequences. logits: f32 [batch][seq_stride][num_classes] (row-major,
 * as Logits.data); seq_lens: tokens to decode per sequence (<= seq_stride;
 * NULL = all seq_stride), like decode()'s sequenceLength argument; biases: the
 * six calibration biases in model/calibration.ts:29-36 order
 * (backgroundStay, backgroundToStart, insideToContinue, insideToEnd,
 * endToBackground, endToStart); tags: u8 [batch][seq_stride] (entries past a
 * sequence's length are left untouched). num_classes must be 33, as the
 * reference requires. Sequences are decoded on up to n_threads host threads
 * (0 = one per host core). Runs on the host only; no device is touched.
 * --------------------------------------------------------------------- */
int pfhip_viterbi_decode(const float* logits, uint32_t batch, uint32_t seq_stride, const uint32_t* seq_lens,
                         uint32_t num_classes, const float* biases, uint8_t* tags, uint32_t n_threads, char* err,
                         size_t err_cap);

/* Library version string. */
const char* pfhip_version(void);

#ifdef __cplusplus
}
#endif
#endif /* PFHIP_H */
