/* biv_hip.h — C ABI of the MI355X (gfx950) backend for biv's qwen35moe
 * mixture-of-experts feed-forward block.
 *
 * The library replaces, for one GPU, the MoE block that biv computes on the
 * CPU in Model::moe (engine/src/model.rs:860-898) and on Metal in
 * MetalEngine::encode_moe (engine/src/metal/mod.rs:2138-2266).  A Rust
 * `hip` backend binds these functions through `extern "C"` declarations of
 * the same names and argument types (pointers as *const / *mut, sizes as
 * i32 / usize), next to the engine's existing backends.
 *
 * Conventions
 *  - Every function returns 0 on success and a negative BIV_HIP_E_* code on
 *    failure; biv_hip_last_error() then describes it.  This maps onto
 *    Error::Backend(String) (engine/src/error.rs:67-68).
 *  - Weights are copied into device memory at upload (biv borrows them from
 *    the mmap'd GGUF, engine/src/ops.rs:14-20; the GPU needs its own copy).
 *    The context owns every upload and frees it in biv_hip_destroy.
 *  - A context is used by one host thread at a time and runs all of its work
 *    on one HIP stream, in submission order.  It takes no locks.  biv's
 *    Engine is not Send/Sync either (engine/src/batch.rs:1-20).
 *  - Results are deterministic: the same inputs give the same bits on every
 *    run (no floating-point atomics; fixed reduction and combine orders).
 */
#ifndef BIV_HIP_H
#define BIV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor types (engine/src/quant.rs:31-48).  The MoE path computes with
 * F32 (router, shared gate), Q8_0, Q4_K, Q6_K and BF16 (experts). */
enum {
    BIV_GGML_F32 = 0,
    BIV_GGML_F16 = 1,
    BIV_GGML_Q8_0 = 8,
    BIV_GGML_Q4_K = 12,
    BIV_GGML_Q6_K = 14,
    BIV_GGML_BF16 = 30,
};

enum {
    BIV_HIP_OK = 0,
    BIV_HIP_E_INVALID = -1, /* bad argument or shape (Error::TensorShape, model.rs:332-340) */
    BIV_HIP_E_TYPE = -2,    /* no kernel for this type (Error::NoKernel, model.rs:341-346) */
    BIV_HIP_E_DEVICE = -3,  /* HIP runtime failure */
    BIV_HIP_E_NOMEM = -4,   /* device allocation failed (Error::OutOfMemory) */
    BIV_HIP_E_FORMAT = -5,  /* malformed GGUF (Error::Truncated, BadMagic, UnsupportedVersion, ...; error.rs:13-25) */
    BIV_HIP_E_IO = -6,      /* a GGUF file cannot be opened or mapped */
    BIV_HIP_E_MISSING = -7, /* GGUF key or tensor absent (Error::MissingKey / MissingTensor, error.rs:28-29) */
    BIV_HIP_E_BUSY = -8,    /* the GPU's no-allocation scratch is held by another context (no counterpart) */
};

/* forward flags */
enum {
    BIV_HIP_ADD = 1, /* x += moe(h), as the caller of Model::ffn does (model.rs:788-790) */
};

typedef struct biv_hip_ctx biv_hip_ctx;
typedef struct biv_hip_weight biv_hip_weight;
typedef struct biv_hip_experts biv_hip_experts;
typedef struct biv_hip_moe biv_hip_moe;

/* A context on HIP device `device` with its own stream.  Replaces the
 * backend construction of MetalEngine::new (engine/src/metal/mod.rs:610-686). */
int biv_hip_create(int device, biv_hip_ctx **out);

/* Frees every weight, layer and scratch buffer of the context. */
void biv_hip_destroy(biv_hip_ctx *ctx);

/* The last error of the context, or of the last failed biv_hip_create when
 * ctx is NULL.  Valid until the next call on the context. */
const char *biv_hip_last_error(const biv_hip_ctx *ctx);

/* Run the context's work on an existing stream (a hipStream_t, e.g. the one
 * a caller times with events) instead of its own; NULL restores its own. */
int biv_hip_set_stream(biv_hip_ctx *ctx, void *stream);

/* Wait for all work submitted on the context's stream. */
int biv_hip_sync(biv_hip_ctx *ctx);

/* Upload one matrix of `rows` rows of `cols` elements in ggml layout
 * (Weight::new, engine/src/ops.rs:22-33): `data` holds rows * row_size(cols)
 * bytes on the host.  Used for the router, the shared expert and its gate.
 * An F32 matrix takes twice its bytes on the device: the rows in the chain
 * layout of the decode router and as given, for the prefill router. */
int biv_hip_upload_weight(biv_hip_ctx *ctx, int ggml_type, size_t cols, size_t rows, const void *data,
                          biv_hip_weight **out);

/* Upload a stack of `n_expert` matrices of `rows` x `cols`: expert e's matrix
 * starts at data + e * stride + offset (Experts::expert, model.rs:207-216;
 * offset selects the up half of a fused ffn_gate_up_exps, model.rs:389-399).
 * `data` is host memory of at least (n_expert - 1) * stride + offset +
 * rows * row_size(cols) bytes. */
int biv_hip_upload_experts(biv_hip_ctx *ctx, int ggml_type, size_t cols, size_t rows, size_t n_expert,
                           const void *data, size_t stride, size_t offset, biv_hip_experts **out);

/* A MoE block (struct Moe, model.rs:229-237) from uploaded parts: router
 * [n_expert x n_embd] (F32), gate/up [n_ff x n_embd] and down [n_embd x n_ff]
 * expert stacks, and the shared expert (gate, up, down, gate_inp) or four
 * NULLs for none.  k = experts per token (n_expert_used).  The layer keeps
 * pointers to the parts, which must outlive it. */
int biv_hip_moe_create(biv_hip_ctx *ctx, const biv_hip_weight *router, const biv_hip_experts *gate,
                       const biv_hip_experts *up, const biv_hip_experts *down, const biv_hip_weight *shared_gate,
                       const biv_hip_weight *shared_up, const biv_hip_weight *shared_down,
                       const biv_hip_weight *gate_inp, int k, biv_hip_moe **out);

/* The block over n tokens: h is [n x n_embd] f32, already normalised (the h of
 * Model::layer, model.rs:788).  out = moe(h), or out += moe(h) with
 * BIV_HIP_ADD.  Host pointers; returns when out is written.  Same result as
 * Model::ffn for a MoE layer (model.rs:853-898). */
int biv_hip_moe_forward(biv_hip_ctx *ctx, const biv_hip_moe *moe, const float *h, int n, float *out,
                        unsigned flags);

/* As biv_hip_moe_forward with device pointers, queued on the context's stream
 * without waiting: the counterpart of encode_moe (metal/mod.rs:2138-2148),
 * which adds into the residual buffer x when flags has BIV_HIP_ADD. */
int biv_hip_moe_forward_device(biv_hip_ctx *ctx, const biv_hip_moe *moe, const float *h_dev, int n, float *out_dev,
                               unsigned flags);

/* biv_hip_moe_forward_device for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops): no counterpart in the reference.
 * It calls no allocator: its scratch is a fixed 48 MiB device buffer of the
 * library, one per GPU, held until the process ends, which fits up to about
 * 350 tokens of a qwen35moe layer (n_embd 2048, n_ff 512, 256 experts, k 8);
 * larger n gives BIV_HIP_E_INVALID.  The buffer is reserved in every
 * process that loads the library and is not counted by
 * biv_hip_device_bytes.  The first context to call this on a GPU holds that
 * GPU's buffer until it is destroyed; another context gets BIV_HIP_E_BUSY.
 * Calls of the holding context that overlap (two streams) race.  Stage
 * timing (biv_hip_set_timing) must be off: it creates events. */
int biv_hip_moe_forward_device_noalloc(biv_hip_ctx *ctx, const biv_hip_moe *moe, const float *h_dev, int n,
                                       float *out_dev, unsigned flags);

/* Debug taps of one forward, host buffers, each optional (NULL to skip).
 * P = n * k routed pairs, in dispatch order: grouped by expert in ascending
 * id, tokens ascending within an expert (the `routed` lists of model.rs:866-873).
 * Rows P .. P + n - 1 of the *_idots and act_* taps are the shared expert's,
 * one per token. */
typedef struct biv_hip_taps {
    int32_t *ids;         /* [n x k] chosen experts, in rank order (route, model.rs:256-268) */
    float *weights;       /* [n x k] their weights */
    float *logits;        /* [n x n_expert] router logits */
    float *shared_logit;  /* [n] gate_inp logit of each token */
    int32_t *pair_token;  /* [P] token of each pair in dispatch order */
    int32_t *pair_expert; /* [P] expert of each pair in dispatch order */
    int32_t *gate_idots;  /* [P + n][n_ff][n_embd / 32] int32 dot of every 32-element block */
    int32_t *up_idots;    /* [P + n][n_ff][n_embd / 32] */
    int8_t *act_q;        /* [P + n][n_ff] the quantised SwiGLU intermediate */
    float *act_d;         /* [P + n][n_ff / 32] its block scales */
    int32_t *down_idots;  /* [P + n][n_embd][n_ff / 32] */
} biv_hip_taps;

/* biv_hip_moe_forward with the debug kernels' taps: the same kernels,
 * instantiated to also store what `taps` asks for.  Host pointers. */
int biv_hip_moe_forward_taps(biv_hip_ctx *ctx, const biv_hip_moe *moe, const float *h, int n, float *out,
                             unsigned flags, const biv_hip_taps *taps);

/* A dense SwiGLU FFN layer, the FFN of biv's `qwen35` (dense) models:
 * Ffn::Dense { gate, up, down } (engine/src/model.rs:239-246), loaded by
 * Loader::ffn (model.rs:377-386).  gate and up [n_ff x n_embd] of one type,
 * down [n_embd x n_ff]; each Q8_0, Q4_K, Q6_K or BF16; n_embd and n_ff
 * multiples of 512.  Uploaded with biv_hip_upload_weight; the layer keeps
 * pointers to them. */
typedef struct biv_hip_dense biv_hip_dense;
int biv_hip_dense_create(biv_hip_ctx *ctx, const biv_hip_weight *gate, const biv_hip_weight *up,
                         const biv_hip_weight *down, biv_hip_dense **out);

/* dense_ffn (model.rs:1118-1126) over n rows of h [n x n_embd] f32:
 * out = down(silu(gate h) * up h), or out += it with BIV_HIP_ADD (the
 * residual add of Model::layer, model.rs:788-790).  Every dot product runs
 * in the reference's x86 accumulation order over the whole row, so the
 * result is Model::ffn's for a dense layer.  Host pointers; returns when out
 * is written. */
int biv_hip_dense_forward(biv_hip_ctx *ctx, const biv_hip_dense *d, const float *h, int n, float *out,
                          unsigned flags);

/* The same with device pointers, queued on the context's stream. */
int biv_hip_dense_forward_device(biv_hip_ctx *ctx, const biv_hip_dense *d, const float *h_dev, int n, float *out_dev,
                                 unsigned flags);

/* Device memory helpers for callers without another allocator. */
int biv_hip_malloc(biv_hip_ctx *ctx, size_t bytes, void **out);
int biv_hip_free(biv_hip_ctx *ctx, void *p);
int biv_hip_memcpy_h2d(biv_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
int biv_hip_memcpy_d2h(biv_hip_ctx *ctx, void *dst, const void *src, size_t bytes);

/* Name/value pairs of what decides the numbers (Engine::numerics,
 * engine/src/engine.rs:42-46), as "name=value;..." into buf. */
int biv_hip_numerics(const biv_hip_ctx *ctx, char *buf, size_t len);

/* Bytes of device memory held by the context's uploads (Engine::device_memory,
 * engine/src/engine.rs:36-40). */
size_t biv_hip_device_bytes(const biv_hip_ctx *ctx);

/* Stage timing for measurement: while enabled, every forward records a HIP
 * event on the context's stream before each of its 6 stages (router with
 * the quantisation of h, or pre-pass and router; route and dispatch sort;
 * gate/up; quantisation of the intermediate; down; combine), a stage being
 * one or more launches or none, and after the last.
 * biv_hip_stage_times waits for the stream, writes the summed milliseconds
 * per stage into ms[0..5] and the number of timed forwards, and forgets
 * them.  The reference times with wall clocks only
 * (src/bench.rs:86-103, examples/bench.rs:22-35). */
int biv_hip_set_timing(biv_hip_ctx *ctx, int enable);
int biv_hip_stage_times(biv_hip_ctx *ctx, double *ms, int n_stages, int *n_forwards);

/* ops::rms_norm (engine/src/ops.rs:136-144) of `rows` rows of n floats in
 * device memory, in place: per row ss = dot_f32(g, g) / n (the x86 32-chain
 * order), scale = 1 / sqrt(ss + eps), v *= scale * w[i].  The norm between
 * stacked MoE layers (post_norm before Model::ffn, model.rs:786-790).  n is
 * a multiple of 32.  Queued on the context's stream. */
int biv_hip_rms_norm(biv_hip_ctx *ctx, float *x_dev, const float *w_dev, int rows, int n, float eps);

/* The feed-forward half of Model::layer for a MoE layer
 * (engine/src/model.rs:788-790), in device memory: h = rms_norm(x, norm, eps)
 * (ops::rms_norm_into), then x += moe(h) (ops::add_inplace), for the n rows of
 * x (n x n_embd floats).  norm_dev holds the layer's post_norm (n_embd
 * floats).  h lives in the context's scratch.  Queued on the context's
 * stream. */
int biv_hip_moe_ffn_step(biv_hip_ctx *ctx, const biv_hip_moe *moe, float *x_dev, const float *norm_dev, float eps,
                         int n);

/* Measurement of one stage alone (index as in biv_hip_stage_times): runs one
 * forward of moes[0] on the n tokens at h_dev (for its routing and
 * dispatch), then launches that stage reps times back to back on the
 * context's stream, layer moes[r % n_moes] at launch r (layers of the same
 * shape and types, e.g. copies in HBM so that weights are not re-read from
 * cache), between two events; writes the milliseconds per launch.  A stage a
 * forward skips (the separate quantisation when the down kernel quantises)
 * measures the empty stream.  No counterpart in the reference, which times
 * whole passes only (src/bench.rs:86-103). */
int biv_hip_time_stage(biv_hip_ctx *ctx, const biv_hip_moe *const *moes, int n_moes, const float *h_dev, int n,
                       float *out_dev, int stage, int reps, double *ms_per_launch);

/* ---- GGUF files (biv's reader: engine/src/gguf.rs, engine/src/model.rs:298-421) ----
 *
 * A GGUF (or the shards of a split one, in order) memory-mapped and parsed
 * as Gguf::from_shards does (gguf.rs:236-306): key/values of every value
 * type, the tensor table, data at general.alignment (32 by default); for a
 * key in several shards the first holds.  The handle keeps the mappings
 * until biv_gguf_close.  A handle is used by one thread at a time. */
typedef struct biv_gguf biv_gguf;

int biv_gguf_open(const char *const *paths, int n_paths, biv_gguf **out);
void biv_gguf_close(biv_gguf *g);
/* The handle's last error, or that of the last failed biv_gguf_open on this
 * thread when g is NULL (Error's Display, error.rs:74-90). */
const char *biv_gguf_last_error(const biv_gguf *g);

/* Metadata values (Gguf::get with Value::as_u64 / as_f32 / as_str,
 * gguf.rs:40-75, 322-330).  BIV_HIP_E_MISSING for an absent key. */
int biv_gguf_get_u64(biv_gguf *g, const char *key, uint64_t *out);
int biv_gguf_get_f32(biv_gguf *g, const char *key, float *out);
int biv_gguf_get_str(biv_gguf *g, const char *key, char *buf, size_t len);

/* The tensor table in file order (Gguf::tensor_order) and Gguf::tensor
 * (gguf.rs:340-350): type, dims in ggml order (dims[0] contiguous; unused
 * dims 1), the mapped bytes and their size. */
int biv_gguf_n_tensors(const biv_gguf *g);
const char *biv_gguf_tensor_name(const biv_gguf *g, int i);
int biv_gguf_tensor(biv_gguf *g, const char *name, int *ggml_type, int *n_dims, uint64_t dims[4], const void **data,
                    size_t *n_bytes);

/* The MoE part of Config (model.rs:70-120) for general.architecture
 * "qwen35moe": n_layer = block_count - nextn_predict_layers, n_embd,
 * expert_count, expert_used_count (1..expert_count), expert and shared
 * expert feed-forward lengths (the shared one 0 when absent), the RMSNorm
 * epsilon. */
typedef struct {
    char arch[32];
    int n_layer, n_embd, n_expert, n_expert_used, n_ff_exp, n_ff_shexp;
    float eps;
} biv_gguf_moe_config;
int biv_gguf_read_moe_config(biv_gguf *g, biv_gguf_moe_config *cfg);

/* Loader::ffn for MoE layer `layer` (model.rs:386-421): checks the shapes of
 * blk.<layer>.ffn_gate_inp (router), ffn_gate_exps + ffn_up_exps or the
 * fused ffn_gate_up_exps (gate rows then up rows per expert, model.rs:
 * 389-399), ffn_down_exps and, when expert_shared_feed_forward_length > 0,
 * ffn_{gate,up,down}_shexp and ffn_gate_inp_shexp (Error::TensorShape as
 * BIV_HIP_E_INVALID), uploads them from the mapping and creates the layer
 * with k = expert_used_count (as biv_hip_moe_create). */
int biv_hip_moe_from_gguf(biv_hip_ctx *ctx, biv_gguf *g, int layer, biv_hip_moe **out);

/* The dense part of Config (model.rs:70-131) for general.architecture
 * "qwen35": n_layer = block_count - nextn_predict_layers, n_embd
 * (embedding_length), n_ff (feed_forward_length), the RMSNorm epsilon. */
typedef struct {
    char arch[32];
    int n_layer, n_embd, n_ff;
    float eps;
} biv_gguf_dense_config;
int biv_gguf_read_dense_config(biv_gguf *g, biv_gguf_dense_config *cfg);

/* Loader::ffn for dense layer `layer` (model.rs:381-386): checks
 * blk.<layer>.ffn_gate and ffn_up [n_embd, n_ff] and ffn_down [n_ff, n_embd]
 * (Error::TensorShape as BIV_HIP_E_INVALID), uploads them from the mapping
 * and creates the layer (as biv_hip_dense_create). */
int biv_hip_dense_from_gguf(biv_hip_ctx *ctx, biv_gguf *g, int layer, biv_hip_dense **out);

#ifdef __cplusplus
}
#endif

#endif /* BIV_HIP_H */
