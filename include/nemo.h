/*
 * libnemo: MI355X (gfx950) Nemotron-3-Embed encoder forward pass behind a
 * plain C ABI. This is the native side of the reference's embedding runtime
 * (src/webgpu/model.ts NemotronWebGPUModel / NemotronExecutionPlan and the
 * EmbeddingRuntime / EmbeddingPlan interfaces of
 * src/webgpu/embedding-engine.ts:7-14). Host bindings (Python ctypes in
 * nemo_amd, the Node-API addon) call exactly these symbols.
 *
 * Conventions: every call returns a nemo_status; on failure
 * nemo_last_error() returns a message for the calling thread (the reference
 * throws an Error with that message). No C++ exception crosses the ABI.
 * Host pointers are copied before a blocking call returns; output buffers
 * are owned by the caller. Pointers documented as "device" are HIP device
 * pointers on the context's device.
 */
#ifndef NEMO_H
#define NEMO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t nemo_status;
#define NEMO_OK 0
#define NEMO_ERR_INVALID 1     /* bad argument, shape or format */
#define NEMO_ERR_MISSING 2     /* a tensor the graph needs was never set */
#define NEMO_ERR_DEVICE 3      /* HIP runtime failure */
#define NEMO_ERR_OOM 4         /* device or pinned host allocation failed */
#define NEMO_ERR_UNSUPPORTED 5 /* valid input this build does not execute */

/* GGML tensor type codes, src/gguf/types.ts:17-23. */
#define NEMO_TYPE_F32 0
#define NEMO_TYPE_F16 1
#define NEMO_TYPE_Q4_0 2
#define NEMO_TYPE_Q4_K 12
#define NEMO_TYPE_Q6_K 14
/* Q4_0 in the wgpack "q4_0-tile32-compact" layout: 20-byte records
 * [f16 d][2 zero bytes][16 nibble bytes] ordered tile (32 rows) -> 32-value
 * block -> row (src/prepacked/format.ts:65-99). Not a GGML type code; the
 * tensor is held and returned as NEMO_TYPE_Q4_0. */
#define NEMO_TYPE_Q4_0_TILE32 258

typedef struct nemo_ctx nemo_ctx;
typedef struct nemo_model nemo_model;
typedef struct nemo_plan nemo_plan;
typedef struct nemo_weight nemo_weight;

/* Model shape. The reference hard-codes these (src/webgpu/model.ts:19-28,
 * src/webgpu/ops.ts:126,186,242,258); here they are parameters so one build
 * runs both the reference dims and other shapes of the same architecture. */
typedef struct nemo_dims {
  int32_t hidden;              /* 2048 */
  int32_t q_heads;             /* 24 */
  int32_t kv_heads;            /* 8 */
  int32_t head_dim;            /* 128 (64 also supported) */
  int32_t intermediate;        /* 6144 */
  int32_t layers;              /* 16 */
  int32_t vocab;               /* 131072 */
  int32_t merge_after_layer;   /* 4: MERGE_AFTER_LAYER, model.ts:26; 0..layers,
                                  where == layers merges just before the pool */
  float rms_epsilon;           /* 1e-5: model.ts:27 */
  float rope_theta;            /* 1e6: model.ts:28 */
  int32_t kv_stride_threshold; /* 2048: ops.ts:258 */
  int32_t kv_stride;           /* 3: ops.ts:258 */
  int32_t kv_dense_before_merge; /* 0: the code's rule (ops.ts:258) in every layer, so a request longer
                                    than the threshold samples keys before the merge too; 1: the rule
                                    README.md:26 states: layers before the merge attend every key, and
                                    merged sequences through the threshold use full attention */
} nemo_dims;

/* Fills the reference model's constants (src/webgpu/model.ts:19-28). */
void nemo_dims_reference(nemo_dims* out);

/* Message of the last failing call on this thread ("" if none). */
const char* nemo_last_error(void);

/* Library version string. */
const char* nemo_version(void);

/* Testing hook, no counterpart in the reference: the calling thread's
 * `checks`-th HIP status check from now on (counting every HIP call the
 * library makes and checks on that thread, launches included) fails as if
 * that call had returned an error, so tests can end an enqueue partway with
 * kernels already queued. 0 turns it off. */
void nemo_debug_fail_after(int32_t checks);

/* Open a context on HIP device `device` (replaces requestWebGPUDevice,
 * src/webgpu/device.ts:6-24). */
nemo_status nemo_init(int32_t device, nemo_ctx** out);
nemo_status nemo_shutdown(nemo_ctx* ctx);

/* ---- model (src/webgpu/model.ts:236-329) -------------------------------- */

nemo_status nemo_model_create(nemo_ctx* ctx, const nemo_dims* dims, nemo_model** out);

/* Upload one tensor (replaces createBufferWithData per tensor,
 * src/webgpu/model.ts:264-266,283-286). `dims` are GGUF dims (ne0 first: a
 * matrix of n rows by k columns is {k, n}). Matrices: NEMO_TYPE_Q4_K,
 * NEMO_TYPE_Q6_K or NEMO_TYPE_Q4_0 raw GGUF blocks, or NEMO_TYPE_Q4_0_TILE32
 * records of a .wgpack (k a multiple of 256 for every matrix type); norms:
 * NEMO_TYPE_F32; token_embd.weight:
 * NEMO_TYPE_Q6_K or NEMO_TYPE_F16. Names are the GGUF names; the fused
 * blk.N.attn_qkv.weight / blk.N.ffn_gate_up.weight may be given directly or
 * as their parts (attn_q/attn_k/attn_v, ffn_gate/ffn_up), fused at finalize
 * like combineQ4 (src/webgpu/model.ts:288-304). */
nemo_status nemo_model_set_tensor(nemo_model* model, const char* name, int32_t ggml_type, const int64_t* dims,
                                  int32_t n_dims, const void* bytes, size_t n_bytes);

/* Fill every tensor with seeded synthetic weights generated on the device:
 * matrices N(0, 0.02) quantized to Q4_K (ffn_down to Q6_K), norm weights 1,
 * token_embd.weight N(0, 0.02) as `embedding_type` (F16 or Q6_K). */
nemo_status nemo_model_synthesize(nemo_model* model, uint64_t seed, int32_t embedding_type);

/* Validate and fuse; required before nemo_plan_create. Errors name the
 * missing or malformed tensor (src/webgpu/model.ts:278,291-292,309,315,318). */
nemo_status nemo_model_finalize(nemo_model* model);

/* Copy a tensor back to the host in its GGUF byte layout. With out == NULL
 * only *n_bytes is written. */
nemo_status nemo_model_get_tensor(nemo_model* model, const char* name, int32_t* ggml_type, int64_t* dims4,
                                  void* out, size_t* n_bytes);

nemo_status nemo_model_destroy(nemo_model* model);

/* ---- execution plan (src/webgpu/model.ts:58-234) ------------------------ */

/* createPlan(batch, sequence) (src/webgpu/model.ts:328): activations for
 * `batch` requests of up to `sequence` tokens (batch <= 64). */
nemo_status nemo_plan_create(nemo_model* model, int32_t batch, int32_t sequence, nemo_plan** out);

/* EmbeddingPlan.run (src/webgpu/model.ts:146-176; src/webgpu/embedding-engine.ts:8):
 * ids[batch * sequence] padded after each request's tokens, lengths[batch]
 * with 1 <= lengths[b] <= sequence; writes out[batch * hidden] float32,
 * L2-normalised, in input order. Blocking. n_ids != batch * sequence fails
 * with 'token buffer does not match execution plan' (model.ts:147). */
nemo_status nemo_plan_run(nemo_plan* plan, const uint32_t* ids, size_t n_ids, const uint32_t* lengths,
                          size_t n_lengths, float* out);

/* Same graph with ids and out as device pointers, enqueued on `stream`
 * (hipStream_t; NULL = the plan's own stream); lengths are host values.
 * Returns once enqueued. Work of the plan enqueued earlier on another stream
 * is waited for on the device first (the runs share the plan's buffers). If
 * the enqueue fails partway, the call drains `stream` before it returns the
 * error, and later calls on the plan still order after what was queued. */
nemo_status nemo_plan_run_device(nemo_plan* plan, const uint32_t* d_ids, const uint32_t* lengths, size_t n_lengths,
                                 float* d_out, void* stream);

/* profile() (src/webgpu/model.ts:178-224): milliseconds per stage, summed
 * over layers, in the order of nemo_profile_stage_name. */
nemo_status nemo_plan_profile(nemo_plan* plan, const uint32_t* ids, size_t n_ids, const uint32_t* lengths,
                              size_t n_lengths, float* stage_ms, int32_t n_stages);
int32_t nemo_profile_stage_count(void);
const char* nemo_profile_stage_name(int32_t index);

/* destroy() (src/webgpu/model.ts:141-144). Waits for a call on the plan
 * that another thread is running, then for all work the plan enqueued (on
 * its own stream or a caller's), then frees it. The caller must not start
 * further calls on the plan, nor have any waiting to start: the host
 * bindings count their runs in flight and destroy once the last settles. */
nemo_status nemo_plan_destroy(nemo_plan* plan);

/* The plan's batch, sequence and the model's hidden width (any pointer may
 * be NULL): a binding sizes the embeddings of a run, batch * hidden floats,
 * from the plan itself. No counterpart in the reference, whose plan object
 * carries these fields (src/webgpu/model.ts:58-74). */
nemo_status nemo_plan_shape(nemo_plan* plan, int32_t* batch, int32_t* sequence, int32_t* hidden);

/* Copy one activation buffer of the last run to the host, for stage-wise
 * parity checks (the reference's buffers of src/webgpu/model.ts:80-94 are
 * debuggable the same way through readF16Buffer, src/main.ts:24-34). Names:
 * "x_full", "norm_full", "x_merged", "norm_merged", "qkv", "q", "k",
 * "attention", "delta" (written only by projections without a K split),
 * "ffn" (f16, packed rows of the last layer that wrote them) and
 * "embeddings" (float). With out == NULL only *n_bytes is
 * written (the buffer's capacity). Blocks until the plan's work is done. */
nemo_status nemo_plan_read_buffer(nemo_plan* plan, const char* name, void* out, size_t* n_bytes);

/* ---- kernel level (src/webgpu/quant-matmul.ts:438-563) ------------------- */

/* Upload one quantized matrix of n rows by k columns (k % 256 == 0) from raw
 * GGUF bytes: QuantMatmulKernel.createRun's weight buffer
 * (src/webgpu/quant-matmul.ts:503-509). Types Q4_K, Q6_K, Q4_0 (GGUF blocks) and
 * NEMO_TYPE_Q4_0_TILE32 (the wgpack records; quant-matmul.ts:99-108). */
nemo_status nemo_weight_create(nemo_ctx* ctx, int32_t ggml_type, int32_t n, int32_t k, const void* bytes,
                               size_t n_bytes, nemo_weight** out);
nemo_status nemo_weight_destroy(nemo_weight* weight);

#define NEMO_MATMUL_AUTO 0     /* GEMV for m <= 160, two-pass where it pays, else the fused GEMM */
#define NEMO_MATMUL_GEMM 1     /* MFMA GEMM decoding W inside the kernel (tiles chosen by size) */
#define NEMO_MATMUL_GEMV 2     /* split-K GEMV, m <= 160 */
#define NEMO_MATMUL_TWO_PASS 3 /* W expanded to f16 scratch (n * k halves, held by the weight),
                                  then an f16 MFMA GEMM; bit-identical to NEMO_MATMUL_GEMM */
#define NEMO_MATMUL_GEMM_MID 4 /* the fused GEMM on 64-row tiles with deep prefetch (the plan's choice
                                  for mid-size m); bit-identical to NEMO_MATMUL_GEMM */
#define NEMO_MATMUL_GEMM_SPLIT 5 /* the 64-row tiles with K split into fp32 partials summed in chunk
                                    order (the plan's choice for 17..64 rows); scratch is held by the
                                    weight and grows on demand */

/* Y[m, n] = f16(X[m, k] W[n, k]^T), fp32 accumulate; d_x f16 [m, k] and d_y
 * f16 [m, n] are device pointers (createRun + dispatch,
 * src/webgpu/quant-matmul.ts:503-563). */
nemo_status nemo_weight_matmul(nemo_weight* weight, const uint16_t* d_x, int32_t m, uint16_t* d_y, int32_t algo,
                               void* stream);

/* Bytes of the per-GPU static scratch that nemo_weight_matmul_static uses
 * (64 MiB): split-K partial sums need splits * m * n * 4 bytes, the two-pass
 * expansion n * k * 2 (a 16384 x 2048 or 2048 x 8192 matrix at most). */
#define NEMO_STATIC_SCRATCH_BYTES 67108864

/* No counterpart in the reference. nemo_weight_matmul for callers that
 * cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc): same algorithms, kernels and
 * bits, but any scratch (the GEMV's and the split-K tiles' fp32 partial
 * sums, the two-pass f16 expansion of W) lives in a static array of
 * NEMO_STATIC_SCRATCH_BYTES that the library holds on each GPU until the
 * process ends; the call allocates and frees nothing. A call whose scratch
 * would exceed that size fails with NEMO_ERR_INVALID before launching
 * anything. Every call on one GPU shares the array: calls that overlap on
 * one GPU (concurrent streams, or host threads) race and must be ordered by
 * the caller. Under HIP graph capture: make one eager call of the same
 * shape and algorithm first (the first call of a kernel sets its LDS size
 * attribute); the captured launches record no memset, and replays equal
 * eager calls bit for bit (tests/test_zz_no_alloc.py). */
nemo_status nemo_weight_matmul_static(nemo_weight* weight, const uint16_t* d_x, int32_t m, uint16_t* d_y,
                                      int32_t algo, void* stream);

/* Decode the uploaded matrix to float32 [n, k] (device pointer); bit-exact
 * with dequantizeQ4KBlock / dequantizeQ6KBlock (src/gguf/quantization.ts:19-74). */
nemo_status nemo_weight_dequantize(nemo_weight* weight, float* d_out, void* stream);

/* Decode raw GGUF blocks at a 16-byte aligned device pointer to float32
 * and/or f16 (either output may be NULL): dequantizeQ4KBlock,
 * dequantizeQ6KBlock, dequantizeQ40Block (src/gguf/quantization.ts:19-74).
 * n_values must be a whole number of blocks. */
nemo_status nemo_dequantize(int32_t ggml_type, const void* d_raw, int64_t n_values, float* d_out_f32,
                            uint16_t* d_out_f16, void* stream);

/* Roofline probe, no counterpart in the reference: the floors the HBM-bound
 * kernels are measured against. bytes == 0 launches one empty kernel (the
 * cost of a launch); otherwise one kernel reads `bytes` (a multiple of 16)
 * at the 16-byte aligned device pointer d_src once, with fully coalesced
 * 16-byte loads, `loads_per_thread` (1, 2, 4 or 8) per thread, and does
 * nothing else: the least time a kernel reading those bytes in one launch
 * takes. d_sink is a device buffer of 256 uint32 the kernel may write. */
nemo_status nemo_probe_stream(const void* d_src, size_t bytes, int32_t loads_per_thread, uint32_t* d_sink,
                              void* stream);

/* ---- offline requantization (src/gguf/quantization.ts:77-131) ------------ */

/* requantizeMatrixToQ40 (src/gguf/quantization.ts:101-131) on the GPU: the
 * raw GGUF bytes of an n x k matrix of type Q4_K, Q6_K or Q4_0 (host memory,
 * n_src bytes) -> n * k / 32 GGUF Q4_0 blocks of 18 bytes written to `out`
 * (host memory, out_bytes). Bit-exact with the reference's JavaScript, which
 * quantizes each 32 values as quantizeQ40Block (:77-98). Errors as the
 * reference: "K=<k> is not divisible by a K-quant block", "source has <n>
 * bytes; expected <m>". scripts/prepack-model.ts:28-36 calls it per matrix. */
nemo_status nemo_requantize_q40(nemo_ctx* ctx, int32_t src_type, const void* src, size_t n_src, int64_t k, int64_t n,
                                void* out, size_t out_bytes);

#ifdef __cplusplus
}
#endif

#endif /* NEMO_H */
