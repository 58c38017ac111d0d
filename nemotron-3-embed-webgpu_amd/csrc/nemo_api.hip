// C ABI of libnemo: context, model (weights), execution plan (activations and
// the 16-layer graph) and kernel-level entry points. Mirrors
// src/webgpu/model.ts (NemotronWebGPUModel, NemotronExecutionPlan) and
// src/webgpu/quant-matmul.ts (QuantMatmulKernel).
#include <math.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/nemo.h"
#include "nemo_common.h"
#include "nemo_ops.h"
#include "nemo_quant.h"
#include "nemo_synth.h"

using namespace nemo;

namespace {

thread_local std::string g_last_error;

struct NemoError : std::runtime_error {
  nemo_status status;
  NemoError(nemo_status s, const std::string& m) : std::runtime_error(m), status(s) {}
};

[[noreturn]] void fail(nemo_status s, const std::string& m) { throw NemoError(s, m); }

// Testing hook (nemo_debug_fail_after): the calling thread's n-th HIP status
// check from now fails as if that call had returned an error.
thread_local int g_fail_after = 0;

void hip_check(hipError_t e, const char* what) {
  if (g_fail_after > 0 && --g_fail_after == 0 && e == hipSuccess)
    fail(NEMO_ERR_DEVICE, std::string(what) + ": injected failure");
  if (e == hipSuccess) return;
  if (e == hipErrorOutOfMemory) fail(NEMO_ERR_OOM, std::string(what) + ": out of device memory");
  fail(NEMO_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

template <typename F>
nemo_status guarded(F&& f) {
  try {
    f();
    g_last_error.clear();
    return NEMO_OK;
  } catch (const NemoError& e) {
    g_last_error = e.what();
    return e.status;
  } catch (const std::bad_alloc&) {
    g_last_error = "host allocation failed";
    return NEMO_ERR_OOM;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return NEMO_ERR_INVALID;
  }
}

// Device allocation owned by a unique_ptr.
struct DevFree {
  void operator()(void* p) const {
    if (p) (void)hipFree(p);
  }
};
using DevPtr = std::unique_ptr<void, DevFree>;

DevPtr dev_alloc(size_t bytes, const char* what) {
  void* p = nullptr;
  if (bytes == 0) bytes = 16;
  hip_check(hipMalloc(&p, bytes), what);
  return DevPtr(p);
}

struct DevTensor {
  int type = -1;
  std::vector<int64_t> dims;
  DevPtr data;   // raw bytes (Q6_K: 208-byte records)
  DevPtr d6;     // Q6_K / Q4_0 matrices: per-block f16 scale (null when stored raw)
  DevPtr gv;     // Q4_K matrices: the GEMV's tiled copy of the blocks (launch_tile_q4k)
  size_t bytes = 0;  // GGUF byte size
  // Gate/up rows reordered per 128-row tile (64 gate rows, then the matching
  // 64 up rows) for the GEMM's SwiGLU epilogue.
  bool gate_up_interleaved = false;
};

// Reorder the rows of a fused gate/up matrix (2F rows: F gate then F up)
// into 128-row tiles of 64 gate rows followed by the matching 64 up rows.
void interleave_rows(DevPtr& buf, size_t row_bytes, int64_t F) {
  DevPtr out = dev_alloc(row_bytes * 2 * F, "interleaved gate/up");
  const size_t chunk = 64 * row_bytes;
  const size_t tiles = (size_t)F / 64;
  hip_check(hipMemcpy2D(out.get(), 2 * chunk, buf.get(), chunk, chunk, tiles, hipMemcpyDeviceToDevice), "interleave");
  hip_check(hipMemcpy2D((uint8_t*)out.get() + chunk, 2 * chunk, (uint8_t*)buf.get() + F * row_bytes, chunk, chunk,
                        tiles, hipMemcpyDeviceToDevice),
            "interleave");
  buf = std::move(out);
}

// Bytes per row of a split matrix's scale array (Q6_K: one f16 per 256
// values; Q4_0: one per 32).
size_t scale_row_bytes(int type, int64_t k) { return type == kQ4_0 ? (size_t)(k / 32) * 2 : (size_t)(k / 256) * 2; }

void interleave_gate_up(DevTensor& t, int64_t F) {
  const int k = (int)t.dims[0];
  interleave_rows(t.data, qweight_row_bytes(t.type, k), F);
  if (t.d6) interleave_rows(t.d6, scale_row_bytes(t.type, k), F);
}

size_t ggml_bytes(int type, const std::vector<int64_t>& dims) {
  int64_t n = 1;
  for (int64_t d : dims) {
    if (d <= 0) fail(NEMO_ERR_INVALID, "tensor dimensions must be positive");
    n *= d;
  }
  switch (type) {
    case kF32: return (size_t)n * 4;
    case kF16: return (size_t)n * 2;
    case kQ4_0:
      if (dims[0] % 32) fail(NEMO_ERR_INVALID, "Q4_0 row length must be a multiple of 32");
      return (size_t)(n / 32) * 18;
    case kQ4_K:
    case kQ6_K:
      if (dims[0] % 256) fail(NEMO_ERR_INVALID, "K-quant row length must be a multiple of 256");
      return (size_t)(n / 256) * (type == kQ4_K ? 144 : 210);
    case NEMO_TYPE_Q4_0_TILE32:
      if (dims.size() != 2 || dims[0] % 32) fail(NEMO_ERR_INVALID, "compact Q4_0 needs [k, n] with k a multiple of 32");
      return (size_t)((dims[1] + 31) / 32) * (size_t)(dims[0] / 32) * 32 * 20;
    default: fail(NEMO_ERR_UNSUPPORTED, "unsupported GGML type " + std::to_string(type));
  }
}

// GGUF Q4_0 blocks (18 bytes: f16 d, 16 nibble bytes), row major, to the
// split layout (see QWeight).
void split_q40(const uint8_t* raw, int64_t nb, std::vector<uint8_t>& nib, std::vector<uint16_t>& d) {
  nib.resize((size_t)nb * 16);
  d.resize((size_t)nb);
  for (int64_t b = 0; b < nb; ++b) {
    d[b] = (uint16_t)(raw[b * 18] | (raw[b * 18 + 1] << 8));
    memcpy(nib.data() + b * 16, raw + b * 18 + 2, 16);
  }
}

// wgpack tile32-compact records (src/prepacked/format.ts:65-99): record of
// row r, 32-value block kb sits at ((r / 32) * kBlocks + kb) * 32 + r % 32,
// 20 bytes [f16 d][2 zero bytes][16 nibble bytes]; to the split layout.
void split_q40_tile32(const uint8_t* rec, int64_t k, int64_t n, std::vector<uint8_t>& nib, std::vector<uint16_t>& d) {
  const int64_t kb_count = k / 32;
  nib.resize((size_t)(n * kb_count) * 16);
  d.resize((size_t)(n * kb_count));
  for (int64_t r = 0; r < n; ++r)
    for (int64_t kb = 0; kb < kb_count; ++kb) {
      const uint8_t* src = rec + (((r / 32) * kb_count + kb) * 32 + r % 32) * 20;
      d[r * kb_count + kb] = (uint16_t)(src[0] | (src[1] << 8));
      memcpy(nib.data() + (r * kb_count + kb) * 16, src + 4, 16);
    }
}

// Split raw Q6_K blocks into 208-byte records + f16 scales (see QWeight).
void split_q6k(const uint8_t* raw, int64_t nb, std::vector<uint8_t>& rec, std::vector<uint16_t>& d) {
  rec.resize((size_t)nb * 208);
  d.resize((size_t)nb);
  for (int64_t b = 0; b < nb; ++b) {
    memcpy(rec.data() + b * 208, raw + b * 210, 208);
    d[b] = (uint16_t)(raw[b * 210 + 208] | (raw[b * 210 + 209] << 8));
  }
}

void upload_tensor(DevTensor& t, int type, const std::vector<int64_t>& dims, const void* bytes, size_t n_bytes,
                   const std::string& name) {
  const size_t expect = ggml_bytes(type, dims);
  if (n_bytes != expect)
    fail(NEMO_ERR_INVALID, name + " has " + std::to_string(n_bytes) + " bytes; expected " + std::to_string(expect));
  t.dims = dims;
  auto put = [&](const std::vector<uint8_t>& rec, const std::vector<uint16_t>& d, const char* what) {
    t.data = dev_alloc(rec.size(), what);
    t.d6 = dev_alloc(d.size() * 2, "block scales");
    hip_check(hipMemcpy(t.data.get(), rec.data(), rec.size(), hipMemcpyHostToDevice), "upload");
    hip_check(hipMemcpy(t.d6.get(), d.data(), d.size() * 2, hipMemcpyHostToDevice), "upload");
  };
  // Q6_K and Q4_0 matrices are split for aligned GEMM loads; the Q6_K token
  // table stays in its raw 210-byte rows (read by the embedding lookup).
  const bool matrix = dims.size() == 2 && name != "token_embd.weight";
  std::vector<uint8_t> rec;
  std::vector<uint16_t> d;
  if (type == NEMO_TYPE_Q4_0_TILE32) {
    split_q40_tile32((const uint8_t*)bytes, dims[0], dims[1], rec, d);
    put(rec, d, "Q4_0 nibbles");
    t.type = kQ4_0;
    t.bytes = (size_t)(dims[0] / 32) * dims[1] * 18;  // GGUF size, as get_tensor returns it
    return;
  }
  t.type = type;
  t.bytes = n_bytes;
  if (type == kQ6_K && matrix) {
    split_q6k((const uint8_t*)bytes, (int64_t)(n_bytes / 210), rec, d);
    put(rec, d, "Q6_K records");
  } else if (type == kQ4_0 && matrix) {
    split_q40((const uint8_t*)bytes, (int64_t)(n_bytes / 18), rec, d);
    put(rec, d, "Q4_0 nibbles");
  } else {
    t.data = dev_alloc(n_bytes, name.c_str());
    hip_check(hipMemcpy(t.data.get(), bytes, n_bytes, hipMemcpyHostToDevice), "upload");
  }
}

QWeight as_qweight(const DevTensor& t) {
  QWeight w;
  w.type = t.type;
  w.k = (int)t.dims[0];
  w.n = (int)t.dims[1];
  w.blocks = (const uint8_t*)t.data.get();
  w.d = (const uint16_t*)t.d6.get();
  w.gv = (const uint8_t*)t.gv.get();
  return w;
}

// The GEMV's tiled copy of a Q4_K, Q6_K or Q4_0 matrix with a multiple of
// 16 rows (as many bytes as the matrix); other matrices are read in place.
void add_gemv_tiles(DevTensor& t) {
  if (t.dims.size() != 2 || t.gv) return;
  const QWeight w = as_qweight(t);
  const size_t bytes = (t.type == kQ4_K || t.type == kQ6_K || t.type == kQ4_0) ? gemv_tile_bytes(w) : 0;
  if (!bytes || (t.type != kQ4_K && !t.d6)) return;
  t.gv = dev_alloc(bytes, "GEMV tiles");
  hip_check(launch_tile_gemv(w, (uint8_t*)t.gv.get(), 0), "GEMV tiles");
  hip_check(hipStreamSynchronize(0), "GEMV tiles");  // plans run on non-blocking streams
}

int merged_length(int sequence) {  // contextualMergedLength, src/webgpu/model.ts:30-32
  const double m = ceil((double)sequence * 0.64);
  return m < 1 ? 1 : (int)m;
}

// Stage names of profile() (src/webgpu/model.ts:198-211).
const char* const kStages[] = {"embedding_norm", "token_merge", "qkv", "rope_attention", "attention_output",
                               "post_attention_norm", "ffn_up_gate", "swiglu", "ffn_down", "post_ffn_norm", "pool"};
constexpr int kNumStages = 11;

}  // namespace

struct nemo_ctx {
  int device = 0;
  void* scratch = nullptr;  // this device's copy of `scratch` (device address)
};

// Device memory of nemo_weight_matmul_static: the split-K partial sums or the
// f16 expansion of one weight. Every GPU the library runs on holds its own
// copy until the process ends, and every call on that GPU shares it. On the
// host the name is only a stand-in for the symbol, never a device address:
// device_scratch() looks up each device's copy once, and calls pass that
// address to the kernels.
static __device__ __align__(256) unsigned char scratch[NEMO_STATIC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static std::map<int, void*> g_scratch;  // device -> address of its `scratch`

// The address of `scratch` on `device`, which must be the current device.
static void* device_scratch(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  const auto it = g_scratch.find(device);
  if (it != g_scratch.end()) return it->second;
  void* ptr = nullptr;
  hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  if (!ptr) fail(NEMO_ERR_DEVICE, "hipGetSymbolAddress(scratch) returned a null address");
  g_scratch[device] = ptr;
  return ptr;
}

struct LayerWeights {
  QWeight qkv, o, gate_up, down;
  // q, k and v of different GGML types (a Q4_K_M file stores attn_v as Q6_K)
  // stay separate: each part writes its column range of the QKV buffer.
  // Empty when `qkv` holds the fused matrix.
  std::vector<std::pair<QWeight, int>> qkv_parts;
  const float* attn_norm = nullptr;
  const float* ffn_norm = nullptr;
};

struct nemo_model {
  nemo_ctx* ctx = nullptr;
  nemo_dims dims{};
  std::map<std::string, DevTensor> tensors;
  bool finalized = false;
  std::vector<LayerWeights> layers;
  const float* output_norm = nullptr;
  int embedding_type = -1;
  const void* embedding = nullptr;
  std::atomic<int> live_plans{0};  // plans are created and destroyed from any thread
};

struct nemo_weight {
  nemo_ctx* ctx = nullptr;
  DevTensor t;
  QWeight w{};
  DevPtr partials;
  DevPtr wexp;  // f16 expansion for the two-pass GEMM, allocated on first use
  DevPtr split_partials;  // split-K sums of NEMO_MATMUL_GEMM_SPLIT, grown on demand
  size_t split_floats = 0;
};

struct nemo_plan {
  nemo_model* model = nullptr;
  int batch = 0, sequence = 0, merged = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
  DevPtr ids, x_full, norm_full, x_red, norm_red, qkv, attn, delta, ffn, out, rope, partials, wexp;
  size_t wexp_halves = 0;
  // f16 expansions of a layer's gate/up and down weights, written by the QKV
  // and O GEMM launches on the CUs their tiles leave idle (see
  // gemm_f16_kernel), so the gate/up and down GEMMs start from them.
  DevPtr wexp_gu, wexp_dn;
  size_t wexp_gu_halves = 0, wexp_dn_halves = 0;
  // Rows of the last layer run (the attention's RoPE positions) and, made
  // on request, its rotated query and key heads.
  Ragged last_rows{};
  DevPtr q, k;
  // Rotated attended keys and transposed values of a pass's long requests
  // (attention's preparation pass), room for attn_keys_cap keys per kv head.
  DevPtr attn_ks, attn_vts;
  int attn_keys_cap = 0;
  uint32_t* h_ids = nullptr;   // pinned staging
  float* h_out = nullptr;
  // Recorded after every enqueue of the plan's work, on the stream it went
  // to (last_stream): the next enqueue on another stream, read_buffer and
  // destroy wait for it, since every run of the plan shares its buffers.
  hipEvent_t done = nullptr;
  hipStream_t last_stream = nullptr;
  ~nemo_plan() {
    if (h_ids) (void)hipHostFree(h_ids);
    if (h_out) (void)hipHostFree(h_out);
    if (done) (void)hipEventDestroy(done);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

// Every enqueue of a plan's work is bracketed by these (plan->mu held): work
// on a stream other than the last one first waits for the plan's previous
// work, and the event then marks the end of the new work.
static void plan_begin(nemo_plan* p, hipStream_t s) {
  if (p->last_stream && p->last_stream != s) hip_check(hipStreamWaitEvent(s, p->done, 0), "hipStreamWaitEvent");
}
// The end mark is recorded however the enqueue ends: a launch that fails
// partway leaves the kernels before it queued on `s`, and later runs on other
// streams, read_buffer and destroy must still wait for them. A failed enqueue
// also drains `s` before the error returns (its queued copies may still read
// the plan's pinned staging, which the next call overwrites), and so does a
// failed record.
struct PlanEnqueue {
  nemo_plan* p;
  hipStream_t s;
  int unwinding;
  PlanEnqueue(nemo_plan* plan, hipStream_t stream)
      : p(plan), s(stream), unwinding(std::uncaught_exceptions()) {
    plan_begin(p, s);
  }
  ~PlanEnqueue() {
    const bool failed = std::uncaught_exceptions() > unwinding;
    const bool recorded = hipEventRecord(p->done, s) == hipSuccess;
    if (recorded) p->last_stream = s;
    if (failed || !recorded) {
      (void)hipStreamSynchronize(s);
      (void)hipGetLastError();
    }
  }
  PlanEnqueue(const PlanEnqueue&) = delete;
  PlanEnqueue& operator=(const PlanEnqueue&) = delete;
};
// Blocks until all of the plan's enqueued work, on any stream, is done.
static void plan_wait(nemo_plan* p) {
  if (p->last_stream) hip_check(hipEventSynchronize(p->done), "hipEventSynchronize");
  if (p->stream) hip_check(hipStreamSynchronize(p->stream), "hipStreamSynchronize");
}

static void set_device(nemo_ctx* ctx) { hip_check(hipSetDevice(ctx->device), "hipSetDevice"); }

static void validate_dims(const nemo_dims& d) {
  if (d.hidden <= 0 || d.hidden % 256) fail(NEMO_ERR_INVALID, "hidden must be a positive multiple of 256");
  if (d.q_heads <= 0 || d.kv_heads <= 0 || d.q_heads % d.kv_heads)
    fail(NEMO_ERR_INVALID, "q_heads must be a positive multiple of kv_heads");
  if (d.head_dim != 64 && d.head_dim != 128) fail(NEMO_ERR_UNSUPPORTED, "head_dim must be 64 or 128");
  if ((d.q_heads * d.head_dim) % 256) fail(NEMO_ERR_INVALID, "q_heads * head_dim must be a multiple of 256");
  if (d.intermediate <= 0 || d.intermediate % 256) fail(NEMO_ERR_INVALID, "intermediate must be a multiple of 256");
  if (d.layers <= 0 || d.merge_after_layer < 0 || d.merge_after_layer > d.layers)
    fail(NEMO_ERR_INVALID, "merge_after_layer must lie in [0, layers]");
  if (d.vocab <= 0) fail(NEMO_ERR_INVALID, "vocab must be positive");
  if (d.kv_stride < 1) fail(NEMO_ERR_INVALID, "kv_stride must be >= 1");
  if (d.kv_dense_before_merge != 0 && d.kv_dense_before_merge != 1)
    fail(NEMO_ERR_INVALID, "kv_dense_before_merge must be 0 or 1");
}

// Every nemo_* definition below takes C linkage from its declaration in nemo.h.

void nemo_dims_reference(nemo_dims* out) {
  if (!out) return;
  out->hidden = 2048;
  out->q_heads = 24;
  out->kv_heads = 8;
  out->head_dim = 128;
  out->intermediate = 6144;
  out->layers = 16;
  out->vocab = 131072;
  out->merge_after_layer = 4;
  out->rms_epsilon = 1e-5f;
  out->rope_theta = 1e6f;
  out->kv_stride_threshold = 2048;
  out->kv_stride = 3;
  out->kv_dense_before_merge = 0;
}

const char* nemo_last_error(void) { return g_last_error.c_str(); }

const char* nemo_version(void) { return "libnemo 0.1 gfx950"; }

void nemo_debug_fail_after(int32_t checks) { g_fail_after = checks > 0 ? checks : 0; }

nemo_status nemo_init(int32_t device, nemo_ctx** out) {
  return guarded([&] {
    if (!out) fail(NEMO_ERR_INVALID, "out is null");
    int count = 0;
    hip_check(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count)
      fail(NEMO_ERR_INVALID, "device " + std::to_string(device) + " out of range (" + std::to_string(count) + ")");
    hip_check(hipSetDevice(device), "hipSetDevice");
    void* dev_scratch = device_scratch(device);
    auto* c = new nemo_ctx;
    c->device = device;
    c->scratch = dev_scratch;
    *out = c;
  });
}

nemo_status nemo_shutdown(nemo_ctx* ctx) {
  return guarded([&] { delete ctx; });
}

nemo_status nemo_model_create(nemo_ctx* ctx, const nemo_dims* dims, nemo_model** out) {
  return guarded([&] {
    if (!ctx || !dims || !out) fail(NEMO_ERR_INVALID, "null argument");
    validate_dims(*dims);
    auto* m = new nemo_model;
    m->ctx = ctx;
    m->dims = *dims;
    *out = m;
  });
}

nemo_status nemo_model_set_tensor(nemo_model* model, const char* name, int32_t ggml_type, const int64_t* dims,
                                  int32_t n_dims, const void* bytes, size_t n_bytes) {
  return guarded([&] {
    if (!model || !name || !dims || n_dims <= 0 || n_dims > 4 || (!bytes && n_bytes))
      fail(NEMO_ERR_INVALID, "invalid tensor arguments");
    if (model->finalized) fail(NEMO_ERR_INVALID, "model is finalized");
    set_device(model->ctx);
    DevTensor t;
    upload_tensor(t, ggml_type, std::vector<int64_t>(dims, dims + n_dims), bytes, n_bytes, name);
    model->tensors[name] = std::move(t);
  });
}

static DevTensor synth_matrix(int type, int64_t k, int64_t n, uint64_t key, hipStream_t s) {
  DevTensor t;
  t.type = type;
  t.dims = {k, n};
  t.bytes = ggml_bytes(type, t.dims);
  const int64_t nb = k / 256 * n;
  if (type == kQ4_K) {
    t.data = dev_alloc(t.bytes, "synthetic Q4_K");
    hip_check(launch_synth_q4k(key, 0.02f, nb, (uint8_t*)t.data.get(), s), "synthesize");
  } else {
    t.data = dev_alloc((size_t)nb * 208, "synthetic Q6_K");
    t.d6 = dev_alloc((size_t)nb * 2, "synthetic Q6_K scales");
    hip_check(launch_synth_q6k(key, 0.02f, nb, (uint8_t*)t.data.get(), (uint16_t*)t.d6.get(), s), "synthesize");
  }
  return t;
}

static DevTensor ones_vector(int64_t n, hipStream_t s) {
  DevTensor t;
  t.type = kF32;
  t.dims = {n};
  t.bytes = (size_t)n * 4;
  t.data = dev_alloc(t.bytes, "norm weight");
  hip_check(launch_fill_f32(1.0f, n, (float*)t.data.get(), s), "synthesize");
  return t;
}

nemo_status nemo_model_synthesize(nemo_model* model, uint64_t seed, int32_t embedding_type) {
  return guarded([&] {
    if (!model) fail(NEMO_ERR_INVALID, "model is null");
    if (model->finalized) fail(NEMO_ERR_INVALID, "model is finalized");
    if (embedding_type != kF16 && embedding_type != kQ6_K)
      fail(NEMO_ERR_INVALID, "embedding type must be F16 or Q6_K");
    set_device(model->ctx);
    const nemo_dims& d = model->dims;
    const int64_t H = d.hidden, QKV = (int64_t)(d.q_heads + 2 * d.kv_heads) * d.head_dim;
    const int64_t QW = (int64_t)d.q_heads * d.head_dim, F = d.intermediate;
    hipStream_t s = nullptr;
    for (int l = 0; l < d.layers; ++l) {
      const std::string p = "blk." + std::to_string(l) + ".";
      model->tensors[p + "attn_qkv.weight"] = synth_matrix(kQ4_K, H, QKV, synth_key(seed, 16 * l + 0), s);
      model->tensors[p + "attn_output.weight"] = synth_matrix(kQ4_K, QW, H, synth_key(seed, 16 * l + 1), s);
      model->tensors[p + "ffn_gate_up.weight"] = synth_matrix(kQ4_K, H, 2 * F, synth_key(seed, 16 * l + 2), s);
      model->tensors[p + "ffn_down.weight"] = synth_matrix(kQ6_K, F, H, synth_key(seed, 16 * l + 3), s);
      model->tensors[p + "attn_norm.weight"] = ones_vector(H, s);
      model->tensors[p + "ffn_norm.weight"] = ones_vector(H, s);
    }
    model->tensors["output_norm.weight"] = ones_vector(H, s);
    DevTensor e;
    e.type = embedding_type;
    e.dims = {H, (int64_t)d.vocab};
    e.bytes = ggml_bytes(embedding_type, e.dims);
    const uint64_t ekey = synth_key(seed, 1u << 20);
    if (embedding_type == kF16) {
      e.data = dev_alloc(e.bytes, "synthetic embedding");
      hip_check(launch_synth_f16(ekey, 0.02f, H * d.vocab, (uint16_t*)e.data.get(), s), "synthesize");
    } else {
      // Q6_K table rows are read raw (210-byte blocks) by the lookup kernel:
      // synthesize split records, then interleave on the host.
      DevTensor tmp = synth_matrix(kQ6_K, H, d.vocab, ekey, s);
      hip_check(hipDeviceSynchronize(), "synthesize");
      const int64_t nb = H / 256 * d.vocab;
      std::vector<uint8_t> rec((size_t)nb * 208), raw((size_t)nb * 210);
      std::vector<uint16_t> dd((size_t)nb);
      hip_check(hipMemcpy(rec.data(), tmp.data.get(), rec.size(), hipMemcpyDeviceToHost), "synthesize");
      hip_check(hipMemcpy(dd.data(), tmp.d6.get(), dd.size() * 2, hipMemcpyDeviceToHost), "synthesize");
      for (int64_t b = 0; b < nb; ++b) {
        memcpy(raw.data() + b * 210, rec.data() + b * 208, 208);
        raw[b * 210 + 208] = (uint8_t)(dd[b] & 0xff);
        raw[b * 210 + 209] = (uint8_t)(dd[b] >> 8);
      }
      e.data = dev_alloc(e.bytes, "synthetic embedding");
      hip_check(hipMemcpy(e.data.get(), raw.data(), raw.size(), hipMemcpyHostToDevice), "synthesize");
    }
    model->tensors["token_embd.weight"] = std::move(e);
    hip_check(hipDeviceSynchronize(), "synthesize");
  });
}

static const DevTensor& need(nemo_model* m, const std::string& name) {
  auto it = m->tensors.find(name);
  if (it == m->tensors.end()) fail(NEMO_ERR_MISSING, "missing tensor " + name);
  return it->second;
}

// Concatenate matrices by rows (combineQ4, src/webgpu/model.ts:288-300).
static void fuse_rows(nemo_model* m, const std::string& name, const std::vector<std::string>& parts) {
  if (m->tensors.count(name)) return;
  std::vector<const DevTensor*> src;
  for (const auto& p : parts) {
    auto it = m->tensors.find(p);
    if (it == m->tensors.end()) fail(NEMO_ERR_MISSING, "missing tensor " + name + " (or its part " + p + ")");
    src.push_back(&it->second);
  }
  const DevTensor& first = *src[0];
  int64_t rows = 0;
  for (auto* t : src) {
    if (t->type != first.type || (t->type != kQ4_K && t->type != kQ6_K && t->type != kQ4_0) || t->dims.size() != 2 ||
        t->dims[0] != first.dims[0]) {
      std::string all;
      for (const auto& p : parts) all += (all.empty() ? "" : ", ") + p;
      fail(NEMO_ERR_INVALID, "cannot combine " + all);
    }
    rows += t->dims[1];
  }
  DevTensor f;
  f.type = first.type;
  f.dims = {first.dims[0], rows};
  f.bytes = ggml_bytes(f.type, f.dims);
  const size_t row_bytes = qweight_row_bytes(f.type, (int)first.dims[0]);
  f.data = dev_alloc(row_bytes * rows, "fused matrix");
  const bool split = first.d6 != nullptr;
  const size_t drow = scale_row_bytes(f.type, first.dims[0]);
  if (split) f.d6 = dev_alloc(drow * rows, "fused scales");
  size_t off = 0, doff = 0;
  for (auto* t : src) {
    const size_t bytes = row_bytes * t->dims[1];
    hip_check(hipMemcpy((uint8_t*)f.data.get() + off, t->data.get(), bytes, hipMemcpyDeviceToDevice), "fuse");
    off += bytes;
    if (split) {
      const size_t db = drow * t->dims[1];
      hip_check(hipMemcpy((uint8_t*)f.d6.get() + doff, t->d6.get(), db, hipMemcpyDeviceToDevice), "fuse");
      doff += db;
    }
  }
  m->tensors[name] = std::move(f);
  for (const auto& p : parts) m->tensors.erase(p);
}

static QWeight matrix(nemo_model* m, const std::string& name, int64_t k, int64_t n) {
  need(m, name);
  DevTensor& t = m->tensors[name];
  if (t.dims.size() != 2) fail(NEMO_ERR_INVALID, "invalid matrix " + name);
  if (t.type != kQ4_K && t.type != kQ6_K && t.type != kQ4_0)
    fail(NEMO_ERR_UNSUPPORTED, "unsupported matrix type " + std::to_string(t.type) + " for " + name);
  if (t.dims[0] != k || t.dims[1] != n)
    fail(NEMO_ERR_INVALID, name + " has dims [" + std::to_string(t.dims[0]) + ", " + std::to_string(t.dims[1]) +
                               "]; expected [" + std::to_string(k) + ", " + std::to_string(n) + "]");
  add_gemv_tiles(t);
  return as_qweight(t);
}

static const float* vec_f32(nemo_model* m, const std::string& name, int64_t n) {
  const DevTensor& t = need(m, name);
  if (t.type != kF32 || t.dims.size() != 1 || t.dims[0] != n)
    fail(NEMO_ERR_INVALID, name + " must be F32 [" + std::to_string(n) + "]");
  return (const float*)t.data.get();
}

nemo_status nemo_model_finalize(nemo_model* model) {
  return guarded([&] {
    if (!model) fail(NEMO_ERR_INVALID, "model is null");
    if (model->finalized) return;
    set_device(model->ctx);
    const nemo_dims& d = model->dims;
    const int64_t H = d.hidden, QKV = (int64_t)(d.q_heads + 2 * d.kv_heads) * d.head_dim;
    const int64_t QW = (int64_t)d.q_heads * d.head_dim, F = d.intermediate;
    std::vector<LayerWeights> layers(d.layers);
    for (int l = 0; l < d.layers; ++l) {
      const std::string p = "blk." + std::to_string(l) + ".";
      const std::string qn = p + "attn_q.weight", kn = p + "attn_k.weight", vn = p + "attn_v.weight";
      const bool mixed_qkv = !model->tensors.count(p + "attn_qkv.weight") && model->tensors.count(qn) &&
                             model->tensors.count(kn) && model->tensors.count(vn) &&
                             (model->tensors[qn].type != model->tensors[kn].type ||
                              model->tensors[qn].type != model->tensors[vn].type);
      if (mixed_qkv) {
        const int64_t KW = (int64_t)d.kv_heads * d.head_dim;
        layers[l].qkv_parts = {{matrix(model, qn, H, QW), 0},
                               {matrix(model, kn, H, KW), (int)QW},
                               {matrix(model, vn, H, KW), (int)(QW + KW)}};
      } else {
        fuse_rows(model, p + "attn_qkv.weight", {qn, kn, vn});
        layers[l].qkv = matrix(model, p + "attn_qkv.weight", H, QKV);
      }
      fuse_rows(model, p + "ffn_gate_up.weight", {p + "ffn_gate.weight", p + "ffn_up.weight"});
      layers[l].o = matrix(model, p + "attn_output.weight", QW, H);
      matrix(model, p + "ffn_gate_up.weight", H, 2 * F);  // validates before reordering
      DevTensor& gu = model->tensors[p + "ffn_gate_up.weight"];
      if (!gu.gate_up_interleaved) {
        interleave_gate_up(gu, F);
        gu.gate_up_interleaved = true;
        gu.gv.reset();  // tiles of the interleaved rows
      }
      add_gemv_tiles(gu);
      layers[l].gate_up = as_qweight(gu);
      layers[l].down = matrix(model, p + "ffn_down.weight", F, H);
      layers[l].attn_norm = vec_f32(model, p + "attn_norm.weight", H);
      layers[l].ffn_norm = vec_f32(model, p + "ffn_norm.weight", H);
    }
    model->output_norm = vec_f32(model, "output_norm.weight", H);
    const DevTensor& e = need(model, "token_embd.weight");
    if ((e.type != kF16 && e.type != kQ6_K) || e.dims.size() != 2 || e.dims[0] != H || e.dims[1] != d.vocab)
      fail(NEMO_ERR_INVALID, "token_embd.weight must be F16 or Q6_K [" + std::to_string(H) + ", " +
                                 std::to_string(d.vocab) + "]");
    model->embedding_type = e.type;
    model->embedding = e.data.get();
    model->layers = std::move(layers);
    model->finalized = true;
  });
}

nemo_status nemo_model_get_tensor(nemo_model* model, const char* name, int32_t* ggml_type, int64_t* dims4, void* out,
                                  size_t* n_bytes) {
  return guarded([&] {
    if (!model || !name || !n_bytes) fail(NEMO_ERR_INVALID, "null argument");
    set_device(model->ctx);
    const DevTensor& t = need(model, name);
    if (ggml_type) *ggml_type = t.type;
    if (dims4)
      for (int i = 0; i < 4; ++i) dims4[i] = i < (int)t.dims.size() ? t.dims[i] : 1;
    if (!out) {
      *n_bytes = t.bytes;
      return;
    }
    if (*n_bytes < t.bytes) fail(NEMO_ERR_INVALID, "output buffer too small");
    hip_check(hipDeviceSynchronize(), "sync");
    if (t.type == kQ6_K && t.d6) {
      const int64_t nb = (int64_t)(t.bytes / 210);
      std::vector<uint8_t> rec((size_t)nb * 208);
      std::vector<uint16_t> dd((size_t)nb);
      hip_check(hipMemcpy(rec.data(), t.data.get(), rec.size(), hipMemcpyDeviceToHost), "download");
      hip_check(hipMemcpy(dd.data(), t.d6.get(), dd.size() * 2, hipMemcpyDeviceToHost), "download");
      uint8_t* o = (uint8_t*)out;
      for (int64_t b = 0; b < nb; ++b) {
        memcpy(o + b * 210, rec.data() + b * 208, 208);
        o[b * 210 + 208] = (uint8_t)(dd[b] & 0xff);
        o[b * 210 + 209] = (uint8_t)(dd[b] >> 8);
      }
    } else if (t.type == kQ4_0 && t.d6) {
      const int64_t nb = (int64_t)(t.bytes / 18);
      std::vector<uint8_t> nib((size_t)nb * 16);
      std::vector<uint16_t> dd((size_t)nb);
      hip_check(hipMemcpy(nib.data(), t.data.get(), nib.size(), hipMemcpyDeviceToHost), "download");
      hip_check(hipMemcpy(dd.data(), t.d6.get(), dd.size() * 2, hipMemcpyDeviceToHost), "download");
      uint8_t* o = (uint8_t*)out;
      for (int64_t b = 0; b < nb; ++b) {
        o[b * 18] = (uint8_t)(dd[b] & 0xff);
        o[b * 18 + 1] = (uint8_t)(dd[b] >> 8);
        memcpy(o + b * 18 + 2, nib.data() + b * 16, 16);
      }
    } else {
      hip_check(hipMemcpy(out, t.data.get(), t.bytes, hipMemcpyDeviceToHost), "download");
    }
    if (t.gate_up_interleaved) {  // back to GGUF row order: gate rows, then up rows
      const int64_t rows = t.dims[1], F = rows / 2;
      const size_t rb = t.bytes / (size_t)rows;
      std::vector<uint8_t> tmp((uint8_t*)out, (uint8_t*)out + t.bytes);
      for (int64_t r = 0; r < rows; ++r) {
        const int64_t tile = r / 128, local = r % 128;
        const int64_t orig = local < 64 ? 64 * tile + local : F + 64 * tile + (local - 64);
        memcpy((uint8_t*)out + orig * rb, tmp.data() + r * rb, rb);
      }
    }
    *n_bytes = t.bytes;
  });
}

nemo_status nemo_model_destroy(nemo_model* model) {
  return guarded([&] {
    if (!model) return;
    if (model->live_plans) fail(NEMO_ERR_INVALID, "model still has live plans");
    set_device(model->ctx);
    delete model;
  });
}

// ---------------------------------------------------------------------------
// Plan
// ---------------------------------------------------------------------------

// RoPE table (src/webgpu/model.ts:95-106), computed in double, stored float:
// [sequence][head_dim/2] pairs of (cos, sin).
static std::vector<float> rope_table(int sequence, int head_dim, double theta) {
  const int pairs = head_dim / 2;
  const double pi = 3.14159265358979323846;
  auto correction = [&](double beta) { return head_dim * log(16384.0 / (beta * 2 * pi)) / (2 * log(theta)); };
  const double lo = floor(correction(32)), hi = ceil(correction(1));
  std::vector<float> v((size_t)sequence * pairs * 2);
  for (int p = 0; p < sequence; ++p)
    for (int i = 0; i < pairs; ++i) {
      const double ramp = 1 - fmin(1.0, fmax(0.0, (i - lo) / fmax(0.001, hi - lo)));
      const double freq = (1.0 / 16) * (1 - ramp) + ramp;
      const double angle = p * pow(theta, -(double)i / pairs) * freq;
      v[((size_t)p * pairs + i) * 2] = (float)cos(angle);
      v[((size_t)p * pairs + i) * 2 + 1] = (float)sin(angle);
    }
  return v;
}

// Whether a pass of m tokens expands a layer's QKV and O weights to f16 in
// one launch before the QKV projection (both single Q4_K matrices on the
// two-pass path; each expansion alone is latency-bound: 5.6 and 5.3 us at
// the benchmark dims).
static bool expand_qkv_o_together(const LayerWeights& w, int m) {
  return m > kGemvMaxM && w.qkv_parts.empty() && w.qkv.type == kQ4_K && w.o.type == kQ4_K &&
         gemm_two_pass(w.qkv, m, gemm_splits(w.qkv, m)) && gemm_two_pass(w.o, m, gemm_splits(w.o, m));
}

nemo_status nemo_plan_create(nemo_model* model, int32_t batch, int32_t sequence, nemo_plan** out) {
  return guarded([&] {
    if (!model || !out) fail(NEMO_ERR_INVALID, "null argument");
    if (!model->finalized) fail(NEMO_ERR_INVALID, "model is not finalized");
    if (batch < 1 || batch > kMaxBatch) fail(NEMO_ERR_INVALID, "batch must be in [1, 64]");
    if (sequence < 1) fail(NEMO_ERR_INVALID, "sequence must be >= 1");
    set_device(model->ctx);
    const nemo_dims& d = model->dims;
    auto p = std::make_unique<nemo_plan>();
    p->model = model;
    p->batch = batch;
    p->sequence = sequence;
    p->merged = merged_length(sequence);
    const size_t tf = (size_t)batch * sequence, tr = (size_t)batch * p->merged;
    const size_t H = d.hidden, QKV = (size_t)(d.q_heads + 2 * d.kv_heads) * d.head_dim;
    const size_t QW = (size_t)d.q_heads * d.head_dim, F = d.intermediate;
    hip_check(hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking), "hipStreamCreate");
    hip_check(hipEventCreateWithFlags(&p->done, hipEventDisableTiming), "hipEventCreate");
    p->ids = dev_alloc(tf * 4, "token ids");
    p->x_full = dev_alloc(tf * H * 2, "full residual stream");
    p->norm_full = dev_alloc(tf * H * 2, "full normalized hidden state");
    p->x_red = dev_alloc(tr * H * 2, "merged residual stream");
    p->norm_red = dev_alloc(tr * H * 2, "merged normalized hidden state");
    p->qkv = dev_alloc(tf * QKV * 2, "query + key + value raw");
    p->attn = dev_alloc(tf * QW * 2, "attention");
    if (sequence > attn_round_keys(d.head_dim)) {
      p->attn_keys_cap = batch * ((sequence + 31) / 32 * 32);
      const size_t halves = (size_t)d.kv_heads * p->attn_keys_cap * d.head_dim;
      p->attn_ks = dev_alloc(halves * 2, "attention keys");
      p->attn_vts = dev_alloc(halves * 2, "attention values (transposed)");
    }
    p->delta = dev_alloc(tf * H * 2, "residual delta");
    p->ffn = dev_alloc(tf * F * 2, "SwiGLU output");
    // fp32 split-K partial sums of the projections that split K.
    size_t partial_floats = 0;
    auto qkv_matrices = [](const LayerWeights& w) {
      std::vector<const QWeight*> v;
      if (w.qkv_parts.empty()) v.push_back(&w.qkv);
      for (const auto& part : w.qkv_parts) v.push_back(&part.first);
      return v;
    };
    for (const LayerWeights& w : model->layers) {
      std::vector<const QWeight*> mats = qkv_matrices(w);
      mats.push_back(&w.o);
      mats.push_back(&w.down);
      for (const QWeight* q : mats) {
        // the largest pass, and the largest below kLargeM (more splits)
        for (const size_t m : {tf, std::min<size_t>(tf, kLargeM - 1)}) {
          const int s = gemm_splits(*q, (int)m);
          if (s > 1) partial_floats = std::max(partial_floats, (size_t)s * m * q->n);
        }
      }
    }
    // Passes of at most kGemvMaxM tokens take the GEMV, whose split counts differ.
    const size_t small_m = std::min<size_t>(tf, kGemvMaxM);
    for (const LayerWeights& w : model->layers) {
      std::vector<const QWeight*> mats = qkv_matrices(w);
      mats.insert(mats.end(), {&w.o, &w.gate_up, &w.down});
      for (const QWeight* q : mats)
        partial_floats = std::max(partial_floats, (size_t)gemv_splits(*q) * small_m * q->n);
    }
    if (partial_floats) p->partials = dev_alloc(partial_floats * 4, "split-K partial sums");
    // f16 expansion of the largest matrix that takes the two-pass GEMM.
    size_t wexp_halves = 0;
    for (const LayerWeights& w : model->layers) {
      std::vector<const QWeight*> mats = qkv_matrices(w);
      mats.insert(mats.end(), {&w.o, &w.gate_up, &w.down});
      for (const size_t m : {tf, std::min<size_t>(tf, kLargeM - 1)}) {
        for (const QWeight* q : mats)
          if (gemm_two_pass(*q, (int)m, gemm_splits(*q, (int)m)))
            wexp_halves = std::max(wexp_halves, (size_t)q->n * q->k);
        if (expand_qkv_o_together(w, (int)m))
          wexp_halves = std::max(wexp_halves, (size_t)w.qkv.n * w.qkv.k + (size_t)w.o.n * w.o.k);
      }
    }
    if (wexp_halves) p->wexp = dev_alloc(wexp_halves * 2, "f16 weight expansion");
    p->wexp_halves = wexp_halves;
    // Room for the gate/up and down expansions that ride on the QKV and O
    // launches (Q4_K / Q6_K matrices that take the two-pass GEMM).
    size_t gu = 0, dn = 0;
    for (const LayerWeights& w : model->layers)
      for (const size_t m : {tf, std::min<size_t>(tf, kLargeM - 1)}) {
        if (m <= (size_t)kGemvMaxM) continue;
        if (side_part_of(w.gate_up, nullptr).type && gemm_two_pass(w.gate_up, (int)m, 1))
          gu = std::max(gu, (size_t)w.gate_up.n * w.gate_up.k);
        if (side_part_of(w.down, nullptr).type && gemm_two_pass(w.down, (int)m, gemm_splits(w.down, (int)m)))
          dn = std::max(dn, (size_t)w.down.n * w.down.k);
      }
    if (gu) p->wexp_gu = dev_alloc(gu * 2, "f16 gate/up expansion");
    if (dn) p->wexp_dn = dev_alloc(dn * 2, "f16 down expansion");
    p->wexp_gu_halves = gu;
    p->wexp_dn_halves = dn;
    p->out = dev_alloc((size_t)batch * H * 4, "embeddings");
    const std::vector<float> table = rope_table(sequence, d.head_dim, d.rope_theta);
    p->rope = dev_alloc(table.size() * 4, "RoPE sin/cos table");
    hip_check(hipMemcpy(p->rope.get(), table.data(), table.size() * 4, hipMemcpyHostToDevice), "upload");
    hip_check(hipHostMalloc((void**)&p->h_ids, tf * 4, hipHostMallocDefault), "pinned ids");
    hip_check(hipHostMalloc((void**)&p->h_out, (size_t)batch * H * 4, hipHostMallocDefault), "pinned output");
    model->live_plans++;
    *out = p.release();
  });
}

nemo_status nemo_plan_destroy(nemo_plan* plan) {
  return guarded([&] {
    if (!plan) return;
    {
      // A run, profile or read of the plan on another thread finishes first
      // (it holds the lock), then everything the plan enqueued, on any stream.
      std::lock_guard<std::mutex> lock(plan->mu);
      set_device(plan->model->ctx);
      plan_wait(plan);
    }
    plan->model->live_plans--;
    delete plan;
  });
}

nemo_status nemo_plan_shape(nemo_plan* plan, int32_t* batch, int32_t* sequence, int32_t* hidden) {
  return guarded([&] {
    if (!plan) fail(NEMO_ERR_INVALID, "null argument");
    if (batch) *batch = plan->batch;
    if (sequence) *sequence = plan->sequence;
    if (hidden) *hidden = plan->model->dims.hidden;
  });
}

nemo_status nemo_plan_read_buffer(nemo_plan* plan, const char* name, void* out, size_t* n_bytes) {
  return guarded([&] {
    if (!plan || !name || !n_bytes) fail(NEMO_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(plan->mu);
    set_device(plan->model->ctx);
    const nemo_dims& d = plan->model->dims;
    const size_t tf = (size_t)plan->batch * plan->sequence, tr = (size_t)plan->batch * plan->merged;
    const size_t H = d.hidden, QKV = (size_t)(d.q_heads + 2 * d.kv_heads) * d.head_dim;
    const size_t QW = (size_t)d.q_heads * d.head_dim, KW = (size_t)d.kv_heads * d.head_dim, F = d.intermediate;
    const std::string n = name;
    const void* src = nullptr;
    size_t bytes = 0;
    if (out) plan_wait(plan);  // the last run may have gone to a caller's stream
    if (n == "x_full") src = plan->x_full.get(), bytes = tf * H * 2;
    else if (n == "norm_full") src = plan->norm_full.get(), bytes = tf * H * 2;
    else if (n == "x_merged") src = plan->x_red.get(), bytes = tr * H * 2;
    else if (n == "norm_merged") src = plan->norm_red.get(), bytes = tr * H * 2;
    else if (n == "qkv") src = plan->qkv.get(), bytes = tf * QKV * 2;
    else if (n == "q" || n == "k") {
      // RoPE of the last layer's query and key heads, as the attention applied it.
      if (!plan->q) plan->q = dev_alloc(tf * QW * 2, "query rope");
      if (!plan->k) plan->k = dev_alloc(tf * KW * 2, "key rope");
      hip_check(launch_rope((const uint16_t*)plan->qkv.get(), (int)QKV, plan->last_rows, (const float*)plan->rope.get(),
                            d.q_heads, d.kv_heads, d.head_dim, (uint16_t*)plan->q.get(), (uint16_t*)plan->k.get(),
                            plan->stream),
                "rope");
      src = n == "q" ? plan->q.get() : plan->k.get();
      bytes = tf * (n == "q" ? QW : KW) * 2;
    }
    else if (n == "attention") src = plan->attn.get(), bytes = tf * QW * 2;
    else if (n == "delta") src = plan->delta.get(), bytes = tf * H * 2;
    else if (n == "ffn") src = plan->ffn.get(), bytes = tf * F * 2;
    else if (n == "embeddings") src = plan->out.get(), bytes = (size_t)plan->batch * H * 4;
    else fail(NEMO_ERR_INVALID, "unknown plan buffer " + n);
    if (!out) {
      *n_bytes = bytes;
      return;
    }
    if (*n_bytes < bytes) fail(NEMO_ERR_INVALID, "output buffer too small");
    hip_check(hipStreamSynchronize(plan->stream), "sync");
    hip_check(hipMemcpy(out, src, bytes, hipMemcpyDeviceToHost), "download");
    *n_bytes = bytes;
  });
}

int32_t nemo_profile_stage_count(void) { return kNumStages; }

const char* nemo_profile_stage_name(int32_t index) {
  return index >= 0 && index < kNumStages ? kStages[index] : "";
}

// Ragged tables of one run: lengths -> source rows; targetLengths
// (src/webgpu/model.ts:226-233) -> merged rows.
static void ragged_tables(nemo_plan* p, const uint32_t* lengths, size_t n_lengths, Ragged& src, Ragged& dst) {
  if (!lengths) fail(NEMO_ERR_INVALID, "lengths is null");
  if ((int)n_lengths != p->batch) fail(NEMO_ERR_INVALID, "lengths do not match execution plan");
  src.count = dst.count = p->batch;
  src.start[0] = dst.start[0] = 0;
  for (int b = 0; b < p->batch; ++b) {
    const uint32_t len = lengths[b];
    if (len < 1 || len > (uint32_t)p->sequence)
      fail(NEMO_ERR_INVALID, "lengths[" + std::to_string(b) + "] = " + std::to_string(len) + " outside [1, " +
                                 std::to_string(p->sequence) + "]");
    src.start[b + 1] = src.start[b] + (int)len;
    dst.start[b + 1] = dst.start[b] + std::min(p->merged, merged_length((int)len));
  }
}

// Enqueue the whole graph (src/webgpu/model.ts:154-168). `mark(stage, begin)`
// brackets stages for profiling.
template <typename Mark>
static void enqueue_graph(nemo_plan* p, const uint32_t* d_ids, const Ragged& src, const Ragged& dst, float* d_out,
                          hipStream_t s, Mark&& mark) {
  nemo_model* m = p->model;
  const nemo_dims& d = m->dims;
  const int H = d.hidden, QKV = (d.q_heads + 2 * d.kv_heads) * d.head_dim, QW = d.q_heads * d.head_dim;
  const int F = d.intermediate;
  uint16_t* x_full = (uint16_t*)p->x_full.get();
  uint16_t* norm_full = (uint16_t*)p->norm_full.get();
  uint16_t* x_red = (uint16_t*)p->x_red.get();
  uint16_t* norm_red = (uint16_t*)p->norm_red.get();
  uint16_t* qkv = (uint16_t*)p->qkv.get();
  uint16_t* attn = (uint16_t*)p->attn.get();
  uint16_t* delta = (uint16_t*)p->delta.get();
  uint16_t* ffn = (uint16_t*)p->ffn.get();
  float* partials = (float*)p->partials.get();
  uint16_t* wexp = (uint16_t*)p->wexp.get();
  const float* rope = (const float*)p->rope.get();

  mark(0, true);
  hip_check(launch_embed(d_ids, p->sequence, src, m->embedding_type, m->embedding, H, d.vocab, x_full, s), "embedding");
  hip_check(launch_rmsnorm(x_full, nullptr, m->layers[0].attn_norm, norm_full, src.start[src.count], H, d.rms_epsilon, s),
            "rmsnorm");
  mark(0, false);
  // Whether layer l's QKV and O weights are expanded together into wexp (QKV,
  // then O), and the layer whose expansion the previous down launch did.
  auto pair_of = [&](int l) {
    const LayerWeights& w = m->layers[l];
    const Ragged& rows = l < d.merge_after_layer ? src : dst;
    return expand_qkv_o_together(w, rows.start[rows.count]) &&
           (size_t)w.qkv.n * w.qkv.k + (size_t)w.o.n * w.o.k <= p->wexp_halves;
  };
  int pair_done = -1;
  for (int l = 0; l < d.layers; ++l) {
    if (l == d.merge_after_layer) {
      mark(1, true);
      hip_check(launch_merge(x_full, src, dst, H, x_red, s), "token merge");
      hip_check(launch_merge(norm_full, src, dst, H, norm_red, s), "token merge");
      mark(1, false);
    }
    const bool full = l < d.merge_after_layer;
    const Ragged& rows = full ? src : dst;
    const int M = rows.start[rows.count];
    uint16_t* x = full ? x_full : x_red;
    uint16_t* norm = full ? norm_full : norm_red;
    const LayerWeights& w = m->layers[l];
    mark(2, true);
    // At most kGemvMaxM tokens: the split-K GEMV (HBM-bound; the MFMA tiles
    // would leave most CUs idle). Each regime's split counts depend on the
    // weight's shape only, and the GEMV's arithmetic per token does not
    // depend on the pass size, so within a regime a token's result does not
    // depend on the rest of the batch.
    const bool small = M <= kGemvMaxM;
    // QKV and O expanded together: QKV at wexp, O after it (by the previous
    // layer's down launch, or by a launch of its own here).
    const bool pair = !small && pair_of(l);
    uint16_t* wexp_o = pair ? wexp + (size_t)w.qkv.n * w.qkv.k : wexp;
    if (pair && pair_done != l)
      hip_check(launch_expand_q4k_pair(w.qkv.blocks, (int64_t)w.qkv.n * (w.qkv.k / 256), wexp, w.o.blocks,
                                       (int64_t)w.o.n * (w.o.k / 256), wexp_o, s),
                "qkv/o expansion");
    // The gate/up and down weights' f16 expansions, when those GEMMs take the
    // two-pass path, ride on earlier GEMM launches of the layer (their
    // workgroups past the tiles; a launch that cannot carry them does them
    // right after).
    const SidePart part_gu =
        !small && (size_t)w.gate_up.n * w.gate_up.k <= p->wexp_gu_halves && gemm_two_pass(w.gate_up, M, 1)
            ? side_part_of(w.gate_up, (uint16_t*)p->wexp_gu.get())
            : SidePart{};
    const int down_splits = small ? 1 : gemm_splits(w.down, M);
    const SidePart part_dn =
        !small && (size_t)w.down.n * w.down.k <= p->wexp_dn_halves && gemm_two_pass(w.down, M, down_splits)
            ? side_part_of(w.down, (uint16_t*)p->wexp_dn.get())
            : SidePart{};
    // The down expansion goes to the gate/up GEMM when that ends with a
    // launch of rows left over from whole rounds (CUs idle there), else to
    // the O launch. The gate/up expansion is shared: its first 3/4 on the
    // QKV launch, the rest on the O launch (16 x 150 tokens, measured with
    // 200-pass runs: 0.6-0.8 % faster per pass than all of it on the QKV
    // launch; 0.55 and 0.85 of it on the QKV launch did less well).
    const bool dn_on_gu = part_dn.type && part_gu.type && gemm_two_pass_tail(w.gate_up, M, 1);
    const int64_t nq = part_gu.nblocks * 3 / 4;
    SideExpand side_q, side_o, side_t;
    side_q.add(side_part_range(part_gu, 0, nq));
    side_o.add(side_part_range(part_gu, nq, part_gu.nblocks - nq));
    (dn_on_gu ? side_t : side_o).add(part_dn);
    // One matrix, or separate q / k / v parts each into its column range.
    auto qkv_proj = [&](const QWeight& wq, int col, const SideExpand* side) {
      const int sp = gemm_splits(wq, M);
      if (small) {
        hip_check(launch_gemv_ex(norm, H, wq, M, kEpiStore, qkv + col, QKV, partials, s), "qkv gemv");
      } else if (sp == 1) {
        hip_check(launch_gemm_ex(norm, H, wq, M, kEpiStore, 1, qkv + col, QKV, s, wexp, pair, side), "qkv matmul");
      } else {
        hip_check(launch_gemm_ex(norm, H, wq, M, kEpiPartial, sp, partials, wq.n, s, wexp, pair, side),
                  "qkv matmul");
        hip_check(launch_reduce_partials(partials, sp, M, wq.n, qkv + col, QKV, s), "qkv reduce");
      }
    };
    const SideExpand* gu_side = side_q.count ? &side_q : nullptr;
    if (w.qkv_parts.empty()) qkv_proj(w.qkv, 0, gu_side);
    for (size_t i = 0; i < w.qkv_parts.size(); ++i)
      qkv_proj(w.qkv_parts[i].first, w.qkv_parts[i].second, i == 0 ? gu_side : nullptr);
    mark(2, false);
    mark(3, true);
    p->last_rows = rows;
    // Requests longer than one staging round of keys: keys rotated and
    // values transposed once per layer instead of once per 32-query tile.
    int longest = 0;
    for (int b = 0; b < rows.count; ++b) longest = std::max(longest, rows.start[b + 1] - rows.start[b]);
    const bool prep = p->attn_ks && longest > attn_round_keys(d.head_dim);
    // Every key before the merge under the README's rule (no request length
    // exceeds INT32_MAX); the plan's key buffers hold every key of a request.
    const int stride_threshold = d.kv_dense_before_merge && full ? INT32_MAX : d.kv_stride_threshold;
    hip_check(launch_attention(qkv, QKV, rope, rows, d.q_heads, d.kv_heads, d.head_dim, stride_threshold,
                               d.kv_stride, attn, s, prep ? (uint16_t*)p->attn_ks.get() : nullptr,
                               prep ? (uint16_t*)p->attn_vts.get() : nullptr, p->attn_keys_cap),
              "attention");
    mark(3, false);
    // Residual projection (O or down) then x += delta; RMSNorm. With a K
    // split, the norm kernel sums the fp32 partials itself.
    auto residual = [&](const uint16_t* in, int ldin, const QWeight& wt, const float* norm_w, int stage,
                        uint16_t* wx, bool expanded, const SideExpand* side) {
      const int splits = small ? gemv_splits(wt) : gemm_splits(wt, M);
      mark(stage, true);
      if (small)
        hip_check(launch_gemv_ex(in, ldin, wt, M, splits == 1 ? kEpiStore : kEpiPartial,
                                 splits == 1 ? (void*)delta : (void*)partials, H, nullptr, s),
                  "residual gemv");
      else if (splits == 1)
        hip_check(launch_gemm_ex(in, ldin, wt, M, kEpiStore, 1, delta, H, s, wx, expanded, side),
                  "residual matmul");
      else  // K split over the tiles: each split's sum stored as f16, half the bytes of fp32 partials
        hip_check(launch_gemm_ex(in, ldin, wt, M, kEpiPartial16, splits, partials, H, s, wx, expanded, side),
                  "residual matmul");
      mark(stage, false);
      mark(stage + 1, true);
      if (splits == 1)
        hip_check(launch_rmsnorm(x, delta, norm_w, norm, M, H, d.rms_epsilon, s), "rmsnorm");
      else if (small)
        hip_check(launch_rmsnorm_partials(x, partials, splits, norm_w, norm, M, H, d.rms_epsilon, s), "rmsnorm");
      else
        hip_check(launch_rmsnorm_partials16(x, (const uint16_t*)partials, splits, norm_w, norm, M, H, d.rms_epsilon,
                                            s),
                  "rmsnorm");
      mark(stage + 1, false);
    };
    residual(attn, QW, w.o, w.ffn_norm, 4, wexp_o, pair, side_o.count ? &side_o : nullptr);
    mark(6, true);  // gate/up GEMM with SwiGLU in its epilogue
    if (small) {
      hip_check(launch_gemv_ex(norm, H, w.gate_up, M, kEpiSwiGLU, ffn, F, partials, s), "gate/up gemv");
    } else if (part_gu.type) {
      hip_check(launch_gemm_ex(norm, H, w.gate_up, M, kEpiSwiGLU, 1, ffn, F, s, part_gu.out, true,
                               side_t.count ? &side_t : nullptr),
                "gate/up matmul");
    } else {
      hip_check(launch_gemm_ex(norm, H, w.gate_up, M, kEpiSwiGLU, 1, ffn, F, s, wexp), "gate/up matmul");
    }
    mark(6, false);
    const float* next = l + 1 < d.layers ? m->layers[l + 1].attn_norm : m->output_norm;
    if (part_dn.type) {
      // The next layer's QKV and O expansion rides on the down launch (its
      // workgroups past the tiles fill the CUs as the tiles finish): that
      // GEMM reads its own expansion, not wexp, which no later kernel of
      // this layer touches.
      SideExpand side_n;
      if (l + 1 < d.layers && pair_of(l + 1)) {
        const LayerWeights& w1 = m->layers[l + 1];
        const SidePart q1 = side_part_of(w1.qkv, wexp), o1 = side_part_of(w1.o, wexp + (size_t)w1.qkv.n * w1.qkv.k);
        if (q1.type && o1.type && side_n.add(q1) && side_n.add(o1)) pair_done = l + 1;
      }
      residual(ffn, F, w.down, next, 8, part_dn.out, true, side_n.count ? &side_n : nullptr);
    } else
      residual(ffn, F, w.down, next, 8, wexp, false, nullptr);
  }
  if (d.merge_after_layer == d.layers) {  // merge after the last layer (models shorter than the reference)
    mark(1, true);
    hip_check(launch_merge(norm_full, src, dst, H, norm_red, s), "token merge");
    mark(1, false);
  }
  mark(10, true);
  hip_check(launch_mean_pool(norm_red, dst, H, d_out, s), "mean pool");
  mark(10, false);
}

static void check_ids_host(nemo_plan* p, const uint32_t* ids, size_t n_ids, const Ragged& src) {
  if (!ids) fail(NEMO_ERR_INVALID, "ids is null");
  if (n_ids != (size_t)p->batch * p->sequence) fail(NEMO_ERR_INVALID, "token buffer does not match execution plan");
  const uint32_t vocab = (uint32_t)p->model->dims.vocab;
  for (int b = 0; b < p->batch; ++b)
    for (int t = 0; t < src.start[b + 1] - src.start[b]; ++t)
      if (ids[(size_t)b * p->sequence + t] >= vocab)
        fail(NEMO_ERR_INVALID, "token id " + std::to_string(ids[(size_t)b * p->sequence + t]) + " outside vocabulary");
}

nemo_status nemo_plan_run(nemo_plan* plan, const uint32_t* ids, size_t n_ids, const uint32_t* lengths,
                          size_t n_lengths, float* out) {
  return guarded([&] {
    if (!plan || !out) fail(NEMO_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(plan->mu);
    set_device(plan->model->ctx);
    Ragged src, dst;
    ragged_tables(plan, lengths, n_lengths, src, dst);
    check_ids_host(plan, ids, n_ids, src);
    const size_t H = plan->model->dims.hidden;
    hipStream_t s = plan->stream;
    {
      PlanEnqueue enqueue(plan, s);
      memcpy(plan->h_ids, ids, n_ids * 4);
      hip_check(hipMemcpyAsync(plan->ids.get(), plan->h_ids, n_ids * 4, hipMemcpyHostToDevice, s), "upload ids");
      enqueue_graph(plan, (const uint32_t*)plan->ids.get(), src, dst, (float*)plan->out.get(), s, [](int, bool) {});
      hip_check(hipMemcpyAsync(plan->h_out, plan->out.get(), (size_t)plan->batch * H * 4, hipMemcpyDeviceToHost, s),
                "readback");
    }
    hip_check(hipStreamSynchronize(s), "run");
    memcpy(out, plan->h_out, (size_t)plan->batch * H * 4);
  });
}

nemo_status nemo_plan_run_device(nemo_plan* plan, const uint32_t* d_ids, const uint32_t* lengths, size_t n_lengths,
                                 float* d_out, void* stream) {
  return guarded([&] {
    if (!plan || !d_ids || !d_out) fail(NEMO_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(plan->mu);
    set_device(plan->model->ctx);
    Ragged src, dst;
    ragged_tables(plan, lengths, n_lengths, src, dst);
    hipStream_t s = stream ? (hipStream_t)stream : plan->stream;
    PlanEnqueue enqueue(plan, s);
    enqueue_graph(plan, d_ids, src, dst, d_out, s, [](int, bool) {});
  });
}

nemo_status nemo_plan_profile(nemo_plan* plan, const uint32_t* ids, size_t n_ids, const uint32_t* lengths,
                              size_t n_lengths, float* stage_ms, int32_t n_stages) {
  return guarded([&] {
    if (!plan || !stage_ms || n_stages < kNumStages) fail(NEMO_ERR_INVALID, "stage_ms needs 11 entries");
    std::lock_guard<std::mutex> lock(plan->mu);
    set_device(plan->model->ctx);
    Ragged src, dst;
    ragged_tables(plan, lengths, n_lengths, src, dst);
    check_ids_host(plan, ids, n_ids, src);
    hipStream_t s = plan->stream;
    // One event pair per stage instance, like the reference's one timestamp
    // pair per compute pass (destroyed however the call ends).
    const int instances = 3 + plan->model->dims.layers * 8;
    std::vector<hipEvent_t> events(2 * instances, nullptr);
    struct EventsFree {
      std::vector<hipEvent_t>& v;
      ~EventsFree() {
        for (auto& e : v)
          if (e) (void)hipEventDestroy(e);
      }
    } events_free{events};
    for (auto& e : events) hip_check(hipEventCreate(&e), "hipEventCreate");
    std::vector<int> names;
    int next = 0;
    {
      PlanEnqueue enqueue(plan, s);
      memcpy(plan->h_ids, ids, n_ids * 4);
      hip_check(hipMemcpyAsync(plan->ids.get(), plan->h_ids, n_ids * 4, hipMemcpyHostToDevice, s), "upload ids");
      enqueue_graph(plan, (const uint32_t*)plan->ids.get(), src, dst, (float*)plan->out.get(), s,
                    [&](int stage, bool begin) {
                      if (begin) {
                        names.push_back(stage);
                        hip_check(hipEventRecord(events[2 * next], s), "hipEventRecord");
                      } else {
                        hip_check(hipEventRecord(events[2 * next + 1], s), "hipEventRecord");
                        ++next;
                      }
                    });
    }
    hip_check(hipStreamSynchronize(s), "profile");
    for (int i = 0; i < n_stages; ++i) stage_ms[i] = 0.f;
    for (int i = 0; i < next; ++i) {
      float ms = 0.f;
      hip_check(hipEventElapsedTime(&ms, events[2 * i], events[2 * i + 1]), "hipEventElapsedTime");
      stage_ms[names[i]] += ms;
    }
  });
}

// ---------------------------------------------------------------------------
// Kernel level
// ---------------------------------------------------------------------------

nemo_status nemo_weight_create(nemo_ctx* ctx, int32_t ggml_type, int32_t n, int32_t k, const void* bytes,
                               size_t n_bytes, nemo_weight** out) {
  return guarded([&] {
    if (!ctx || !out || !bytes) fail(NEMO_ERR_INVALID, "null argument");
    if (ggml_type != kQ4_K && ggml_type != kQ6_K && ggml_type != kQ4_0 && ggml_type != NEMO_TYPE_Q4_0_TILE32)
      fail(NEMO_ERR_UNSUPPORTED, "weight type must be Q4_K, Q6_K, Q4_0 or compact Q4_0");
    if (k <= 0 || k % 256 != 0) fail(NEMO_ERR_INVALID, "quantized matmul K must be divisible by 256");
    if (n <= 0) fail(NEMO_ERR_INVALID, "n must be positive");
    set_device(ctx);
    auto w = std::make_unique<nemo_weight>();
    w->ctx = ctx;
    upload_tensor(w->t, ggml_type, {k, n}, bytes, n_bytes, "weight");
    add_gemv_tiles(w->t);
    w->w = as_qweight(w->t);
    const size_t pf = gemv_partials_floats(w->w, kGemvMaxM);
    if (pf) w->partials = dev_alloc(pf * 4, "GEMV partials");
    *out = w.release();
  });
}

nemo_status nemo_weight_destroy(nemo_weight* weight) {
  return guarded([&] {
    if (!weight) return;
    set_device(weight->ctx);
    hip_check(hipDeviceSynchronize(), "sync");
    delete weight;
  });
}

// The kernels nemo_weight_matmul runs for (w, m, algo), and the scratch they
// need: fp32 partial sums (GEMV with K split, split-K 64-row tiles) or the
// f16 expansion of W (two-pass).
enum MatmulKind { kMmGemv, kMmMid, kMmSplit, kMmTwoPass, kMmFused };
struct MatmulChoice {
  MatmulKind kind;
  int splits;
  size_t scratch_bytes;
};

static MatmulChoice choose_matmul(const QWeight& w, int m, int algo) {
  if (m < 1) fail(NEMO_ERR_INVALID, "m must be positive");
  if (algo < 0 || algo > 5) fail(NEMO_ERR_INVALID, "unknown matmul algorithm");
  const bool gemv = algo == NEMO_MATMUL_GEMV || (algo == NEMO_MATMUL_AUTO && m <= kGemvMaxM);
  if (gemv) {
    if (m > kGemvMaxM) fail(NEMO_ERR_INVALID, "GEMV takes m <= " + std::to_string(kGemvMaxM));
    return {kMmGemv, gemv_splits(w), gemv_partials_floats(w, m) * 4};
  }
  if (algo == NEMO_MATMUL_GEMM_MID) return {kMmMid, 1, 0};
  if (algo == NEMO_MATMUL_GEMM_SPLIT) {
    const int sp = mid_splits(w);
    return sp == 1 ? MatmulChoice{kMmMid, 1, 0} : MatmulChoice{kMmSplit, sp, (size_t)sp * m * w.n * 4};
  }
  if (algo == NEMO_MATMUL_TWO_PASS || (algo == NEMO_MATMUL_AUTO && gemm_two_pass(w, m, 1)))
    return {kMmTwoPass, 1, (size_t)w.n * w.k * 2};
  return {kMmFused, 1, 0};
}

// Launch `c` on stream s; `scratch` holds at least c.scratch_bytes.
static void run_matmul(const MatmulChoice& c, const QWeight& w, const uint16_t* d_x, int m, uint16_t* d_y,
                       void* scratch, hipStream_t s) {
  switch (c.kind) {
    case kMmGemv:
      hip_check(launch_gemv(d_x, w.k, w, d_y, w.n, m, (float*)scratch, s), "gemv");
      break;
    case kMmMid:
      hip_check(launch_gemm_mid(d_x, w.k, w, m, kEpiStore, 1, d_y, w.n, s), "gemm");
      break;
    case kMmSplit:
      hip_check(launch_gemm_mid(d_x, w.k, w, m, kEpiPartial, c.splits, scratch, w.n, s), "gemm");
      hip_check(launch_reduce_partials((float*)scratch, c.splits, m, w.n, d_y, w.n, s), "reduce");
      break;
    case kMmTwoPass:
      hip_check(launch_gemm_two_pass(d_x, w.k, w, m, d_y, w.n, (uint16_t*)scratch, s), "two-pass gemm");
      break;
    case kMmFused:
      hip_check(launch_gemm(d_x, w.k, w, d_y, w.n, m, s), "gemm");
      break;
  }
}

nemo_status nemo_weight_matmul(nemo_weight* weight, const uint16_t* d_x, int32_t m, uint16_t* d_y, int32_t algo,
                               void* stream) {
  return guarded([&] {
    if (!weight || !d_x || !d_y) fail(NEMO_ERR_INVALID, "null argument");
    const QWeight& w = weight->w;
    const MatmulChoice c = choose_matmul(w, m, algo);
    set_device(weight->ctx);
    hipStream_t s = (hipStream_t)stream;
    void* scratch_buf = nullptr;
    if (c.kind == kMmGemv) {
      scratch_buf = weight->partials.get();  // sized for kGemvMaxM rows at create
    } else if (c.kind == kMmSplit) {
      const size_t need = c.scratch_bytes / 4;
      if (need > weight->split_floats) {
        if (s) hip_check(hipStreamSynchronize(s), "sync");
        weight->split_partials.reset();
        weight->split_partials = dev_alloc(need * 4, "split-K partial sums");
        weight->split_floats = need;
      }
      scratch_buf = weight->split_partials.get();
    } else if (c.kind == kMmTwoPass) {
      if (!weight->wexp) weight->wexp = dev_alloc(c.scratch_bytes, "f16 weight expansion");
      scratch_buf = weight->wexp.get();
    }
    run_matmul(c, w, d_x, m, d_y, scratch_buf, s);
  });
}

nemo_status nemo_weight_matmul_static(nemo_weight* weight, const uint16_t* d_x, int32_t m, uint16_t* d_y,
                                      int32_t algo, void* stream) {
  return guarded([&] {
    if (!weight || !d_x || !d_y) fail(NEMO_ERR_INVALID, "null argument");
    const QWeight& w = weight->w;
    const MatmulChoice c = choose_matmul(w, m, algo);
    if (c.scratch_bytes > (size_t)NEMO_STATIC_SCRATCH_BYTES)
      fail(NEMO_ERR_INVALID, "this matmul needs " + std::to_string(c.scratch_bytes) +
                                 " bytes of scratch; the static scratch holds " +
                                 std::to_string((size_t)NEMO_STATIC_SCRATCH_BYTES));
    set_device(weight->ctx);
    // Every kernel writes each scratch element it later reads (one slot per
    // K split, or the whole expansion), so nothing needs clearing first.
    run_matmul(c, w, d_x, m, d_y, weight->ctx->scratch, (hipStream_t)stream);
  });
}

nemo_status nemo_weight_dequantize(nemo_weight* weight, float* d_out, void* stream) {
  return guarded([&] {
    if (!weight || !d_out) fail(NEMO_ERR_INVALID, "null argument");
    set_device(weight->ctx);
    hip_check(launch_dequant_weight(weight->w, d_out, (hipStream_t)stream), "dequantize");
  });
}

nemo_status nemo_dequantize(int32_t ggml_type, const void* d_raw, int64_t n_values, float* d_out_f32,
                            uint16_t* d_out_f16, void* stream) {
  return guarded([&] {
    if (!d_raw || (!d_out_f32 && !d_out_f16)) fail(NEMO_ERR_INVALID, "null argument");
    if (((uintptr_t)d_raw & 15) != 0) fail(NEMO_ERR_INVALID, "raw blocks must be 16-byte aligned");
    const int per = ggml_type == kQ4_0 ? 32 : 256;
    if (ggml_type != kQ4_K && ggml_type != kQ6_K && ggml_type != kQ4_0)
      fail(NEMO_ERR_UNSUPPORTED, "dequantize supports Q4_0, Q4_K and Q6_K");
    if (n_values < 0 || n_values % per) fail(NEMO_ERR_INVALID, "n_values is not a whole number of blocks");
    hip_check(launch_dequant_raw(ggml_type, (const uint8_t*)d_raw, n_values / per, d_out_f32, d_out_f16,
                                 (hipStream_t)stream),
              "dequantize");
  });
}


nemo_status nemo_probe_stream(const void* d_src, size_t bytes, int32_t loads_per_thread, uint32_t* d_sink,
                              void* stream) {
  return guarded([&] {
    if (bytes == 0) {
      hip_check(launch_probe_empty((hipStream_t)stream), "empty launch");
      return;
    }
    if (!d_src || !d_sink) fail(NEMO_ERR_INVALID, "null argument");
    if (bytes % 16 || ((uintptr_t)d_src & 15)) fail(NEMO_ERR_INVALID, "the probe reads whole 16-byte vectors");
    if (loads_per_thread != 1 && loads_per_thread != 2 && loads_per_thread != 4 && loads_per_thread != 8)
      fail(NEMO_ERR_INVALID, "loads_per_thread must be 1, 2, 4 or 8");
    hip_check(launch_probe_stream(d_src, (int64_t)bytes, loads_per_thread, d_sink, (hipStream_t)stream),
              "streaming probe");
  });
}

nemo_status nemo_requantize_q40(nemo_ctx* ctx, int32_t src_type, const void* src, size_t n_src, int64_t k, int64_t n,
                                void* out, size_t out_bytes) {
  return guarded([&] {
    if (!ctx || !src || !out) fail(NEMO_ERR_INVALID, "null argument");
    if (src_type != kQ4_K && src_type != kQ6_K && src_type != kQ4_0)
      fail(NEMO_ERR_UNSUPPORTED, "requantization reads Q4_K, Q6_K or Q4_0");
    if (k <= 0 || n <= 0) fail(NEMO_ERR_INVALID, "k and n must be positive");
    if (k % 256) fail(NEMO_ERR_INVALID, "K=" + std::to_string(k) + " is not divisible by a K-quant block");
    const size_t expect = src_type == kQ4_0 ? (size_t)n * (k / 32) * 18 : (size_t)n * (k / 256) * (src_type == kQ4_K ? 144 : 210);
    if (n_src != expect)
      fail(NEMO_ERR_INVALID, "source has " + std::to_string(n_src) + " bytes; expected " + std::to_string(expect));
    const size_t need = (size_t)n * (k / 32) * 18;
    if (out_bytes < need) fail(NEMO_ERR_INVALID, "output needs " + std::to_string(need) + " bytes");
    set_device(ctx);
    DevPtr d_src = dev_alloc(n_src, "requantize source");
    DevPtr d_out = dev_alloc(need, "requantize output");
    hip_check(hipMemcpy(d_src.get(), src, n_src, hipMemcpyHostToDevice), "upload");
    hip_check(launch_requant_q40(src_type, (const uint8_t*)d_src.get(), k, n, (uint8_t*)d_out.get(), nullptr),
              "requantize");
    hip_check(hipMemcpy(out, d_out.get(), need, hipMemcpyDeviceToHost), "download");
  });
}
