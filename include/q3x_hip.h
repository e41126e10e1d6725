/*
 * q3x_hip.h -- C ABI of the MI355X (gfx950) quantized-matmul backend.
 *
 * Drop-in boundary for qwen3x's quantized weight matmul.  Weights keep the
 * reference's llama.cpp-compatible 32-element block layouts:
 *   Q8_0 block (34 B): uint16 fp16 scale d, int8 q[32];  w = d * q
 *     (reference q8.h:10-15, arch/cpu.cpp:55-63)
 *   Q4_0 block (18 B): uint16 fp16 scale d, uint8 nib[16]; element j < 16 is
 *     the low nibble of nib[j], element j >= 16 the high nibble of nib[j-16];
 *     w = d * (nibble - 8)  (reference q4.h:10-23, arch/cpu.cpp:81-90)
 * A matrix W[rows, cols] is row-major, each row cols/32 contiguous blocks with
 * no padding; an expert pool W[E, rows, cols] is E such matrices back to back
 * (stride quantized_bytes(rows, cols); reference engine.cpp:214-224).
 * Activations, accumulators and outputs are FP32.
 *
 * Conventions (all entry points):
 *   - every pointer except `bytes` outputs is a DEVICE pointer;
 *   - calls are asynchronous on `stream` (0 = the null stream) and enqueue
 *     nothing when they return an error;
 *   - no entry point allocates, frees, synchronises or keeps state; the MoE
 *     and split-GEMM workspaces are caller-owned; calls are reentrant;
 *   - results are deterministic: no atomics on accumulation paths, fixed
 *     reduction order per shape;
 *   - return Q3X_HIP_OK, or a negative code (arguments are validated before
 *     any device work, so invalid calls touch no memory).
 * The reference's CUDA backend aborts on error (engine.cu:48-56); this ABI
 * returns codes instead so a caller may wrap them in its own assert.
 */
#ifndef Q3X_HIP_H
#define Q3X_HIP_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Matrix type numbering of the reference's model_config.h:16-20. */
enum {
    Q3X_HIP_MATRIX_BF16 = 0,
    Q3X_HIP_MATRIX_Q8_0 = 1,
    Q3X_HIP_MATRIX_Q4_0 = 2,
};

enum {
    Q3X_HIP_OK = 0,
    Q3X_HIP_EINVAL = -1,   /* bad pointer, shape, type or size */
    Q3X_HIP_ERUNTIME = -2, /* a HIP launch or query failed */
    Q3X_HIP_ENOTSUP = -3,  /* valid request this backend does not handle
                              (BF16 matrices: the caller keeps its own path,
                              as with arch/cpu.cpp try_mv returning false) */
};

/* Human-readable name of a return code (static string). */
const char* q3x_hip_strerror(int code);

/* Exact byte size of a Q8_0/Q4_0 matrix.  Mirrors arch/cpu.cpp:161-179
 * (quantized_bytes): rejects BF16/unknown types, rows <= 0, cols <= 0,
 * cols % 32 != 0 and size_t overflow with Q3X_HIP_EINVAL, leaving *bytes
 * untouched. */
int q3x_hip_quantized_bytes(uint32_t type, int rows, int cols, size_t* bytes);

/* y[rows] = W[rows, cols] x[cols]        (accumulate == 0)
 * y[rows] += W[rows, cols] x[cols]       (accumulate != 0)
 * Replaces the CUDA backend's mv() and mv_add() (arch/cuda/engine.cu:1531,
 * 1547; kernels mv_q8_kernel / mv_add_q8_kernel / mv_q4_kernel /
 * mv_add_q4_kernel :574-612) and the CPU try_mv (arch/cpu.cpp:192). */
int q3x_hip_mv(const void* w, uint32_t type, int rows, int cols,
               const float* x, float* y, int accumulate, hipStream_t stream);

/* One matrix of a q3x_hip_mv_multi call: out[rows] (+)= W[rows, cols] x. */
typedef struct q3x_hip_mv_item {
    const void* weight;  /* device, row-major [rows, cols/32] blocks */
    int rows;
    float* out;          /* device, out[rows] */
    int accumulate;      /* nonzero: out += W x */
} q3x_hip_mv_item;

#define Q3X_HIP_MV_MULTI_MAX 8

/* Several matrices of one type and width applied to the same input x, in one
 * launch: items[i].out (+)= items[i].W x for i < count (1..8).  Replaces the
 * CUDA backend's projection helpers attention_projections (q, k, v),
 * ffn_projections (gate, up) and delta_projections (qkv, z, a, b)
 * (arch/cuda/engine.cu:1599-1661), which issue one mv() per matrix for Q8_0.
 * Results equal q3x_hip_mv on each item bit for bit. */
int q3x_hip_mv_multi(const q3x_hip_mv_item* items, int count, uint32_t type, int cols,
                     const float* x, hipStream_t stream);

/* Y[count, rows] (+)= X[count, cols] W[rows, cols]^T, row-major X and Y.
 * Replaces batch_mv() (arch/cuda/engine.cu:1568; batch_mv_q8_kernel :761),
 * and adds the Q4_0 case the CUDA backend lacks (engine.cu:1580).  `count`
 * is unbounded (the reference chunks prefill at 256 tokens, engine.cu:45). */
int q3x_hip_gemm(const void* w, uint32_t type, int rows, int cols,
                 const float* X, int count, float* Y, int accumulate,
                 hipStream_t stream);

/* Bytes of caller-owned workspace with which q3x_hip_gemm_ws splits the K
 * dimension of this GEMM over workgroups (0: it would not split).  For the
 * same shape and arguments as q3x_hip_gemm, with a workspace of at least
 * q3x_hip_gemm_workspace_bytes(type, rows, cols, count) bytes (16-byte
 * aligned; smaller or null runs q3x_hip_gemm's launch): a launch of few
 * output tiles over a long K (e.g. 512 tokens x 5120 rows x 17408 columns)
 * then fills the chip, each tile's K ranges summed by a second launch in K
 * order.  Deterministic; the sums run in another order than q3x_hip_gemm's,
 * within the same tolerance against the reference.  The workspace holds the
 * partial sums from the first launch to the second, so calls that share one
 * must be ordered (e.g. issued on one stream).  Same role as
 * q3x_hip_gemm (batch_mv, arch/cuda/engine.cu:1568); no counterpart of its
 * own in the reference. */
size_t q3x_hip_gemm_workspace_bytes(uint32_t type, int rows, int cols, int count);
int q3x_hip_gemm_ws(const void* w, uint32_t type, int rows, int cols,
                    const float* X, int count, float* Y, int accumulate,
                    void* workspace, size_t workspace_bytes, hipStream_t stream);

/* out[nrows, cols] = dequantised rows [row0, row0 + nrows) of W, bit-exact
 * with the reference's embed (arch/cpu.cpp:55-63, 81-90; CUDA embed_q8_kernel
 * / embed_q4_kernel engine.cu:490-517, batch_embed_q8_kernel :701). */
int q3x_hip_dequant(const void* w, uint32_t type, int cols, int row0, int nrows,
                    float* out, hipStream_t stream);

/* Per-token router: softmax over `experts` logits, top_k sequential argmax
 * (strict '>', lowest index wins ties), weights renormalised over the
 * selection.  logits [tokens, experts]; ids, weights [tokens, top_k].
 * Exact: the softmax repeats the reference's operations (exp with the host
 * libm's expf arithmetic, the total added in expert order, correctly rounded
 * divisions), so ids and weights equal the reference's bit for bit.
 * Replaces router_top_k (engine.cpp:377-405; router_top_k_kernel
 * engine.cu:1153-1184, which runs one thread for one token).
 * Requires 1 <= top_k <= min(experts, 8) and experts <= 1024. */
int q3x_hip_router_topk(const float* logits, int tokens, int experts, int top_k,
                        int* ids, float* weights, hipStream_t stream);

/* Bytes of caller-owned workspace q3x_hip_moe_routed needs. */
size_t q3x_hip_moe_workspace_bytes(int tokens, int experts, int top_k, int H, int I);

/* Routed experts: for every token t,
 *   Y[t] (+)= sum_{slot < top_k} weights[t, slot] * Down_e (silu(G_e X[t]) * U_e X[t])
 * with e = ids[t, slot], G_e / U_e rows [0, I) / [I, 2I) of gate_up[e], in
 * slot order from zero (engine.cpp:406-420; CUDA expert_gate_up_q4_kernel,
 * expert_swiglu_kernel, expert_down_weighted_q4_kernel engine.cu:1186-1250).
 * gate_up: [experts, 2I, H], down: [experts, H, I], type Q4_0 or Q8_0.
 * tokens == 1 runs fused matvecs (decode); tokens > 1 groups the (token,
 * slot) pairs by expert and runs the experts' tiles as grouped GEMMs on the
 * bf16 matrix cores, three exact bf16 products per FP32 product (FP32 sums).
 * ids outside [0, experts) contribute nothing (as engine.cu:1198, 1235). */
int q3x_hip_moe_routed(const void* gate_up, const void* down, uint32_t type,
                       int experts, int H, int I, const float* X, int tokens,
                       const int* ids, const float* weights, int top_k, float* Y,
                       int accumulate, void* workspace, size_t workspace_bytes,
                       hipStream_t stream);

/* Router and routed experts in one call: ids / weights ([tokens, top_k],
 * device, written) = q3x_hip_router_topk(logits [tokens, experts]), then
 * q3x_hip_moe_routed with them -- the reference's decode sequence
 * router_top_k_kernel + expert kernels (engine.cu:1153-1250, 1711-1726).
 * top_k <= 8.  One token takes two launches: the gate/up matvec routes the
 * token itself (every workgroup runs the router on the logits, workgroup 0
 * stores ids / weights) and stores h = silu(g) * u, then the down launch
 * combines the slots; results equal the two calls' bit for bit.  Same
 * workspace as q3x_hip_moe_routed. */
int q3x_hip_moe_routed_logits(const void* gate_up, const void* down, uint32_t type,
                              int experts, int H, int I, const float* X, int tokens,
                              const float* logits, int top_k, int* ids, float* weights,
                              float* Y, int accumulate, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);

/* Size of the library's static per-device scratch that
 * q3x_hip_moe_routed_noalloc runs on: 32 MiB holds the workspace of 256
 * tokens at the 35B-A3B expert shape (H 2048, I 512, top 8), the reference's
 * prefill chunk (engine.cu:45). */
#define Q3X_HIP_NOALLOC_SCRATCH_BYTES (32u << 20)

enum {
    Q3X_HIP_ESCRATCH = -5,  /* request needs more workspace than
                               Q3X_HIP_NOALLOC_SCRATCH_BYTES */
};

/* q3x_hip_moe_routed without a workspace argument, for callers that cannot
 * allocate (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  Same arguments,
 * kernels and results as q3x_hip_moe_routed, run on a workspace the library
 * holds in a static __device__ array of Q3X_HIP_NOALLOC_SCRATCH_BYTES per
 * device (held until the process ends); the call allocates and frees
 * nothing.  Returns Q3X_HIP_ESCRATCH, touching nothing, when
 * q3x_hip_moe_workspace_bytes(tokens, experts, top_k, H, I) exceeds that
 * size.  Runs on the current device (the stream's).  Every call on a device
 * shares that device's scratch: calls that overlap on one device (different
 * streams, or threads without ordering) race; calls ordered on one stream
 * do not.  The first call on a device looks the scratch address up
 * (hipGetSymbolAddress), so make one call before capturing a graph. */
int q3x_hip_moe_routed_noalloc(const void* gate_up, const void* down, uint32_t type,
                               int experts, int H, int I, const float* X, int tokens,
                               const int* ids, const float* weights, int top_k, float* Y,
                               int accumulate, hipStream_t stream);

/* The weights of one MoE layer (the reference's MoeWeights, engine.cu:97-101,
 * engine.cpp:53-57; shapes as model.bin lays them out, engine.cpp:543-550).
 * Every pointer is a device pointer; the struct itself is read on the host. */
typedef struct q3x_hip_moe_layer_weights {
    const void* router;       /* BF16 [experts, H] (mlp.gate), 16-byte aligned */
    const void* gate_up;      /* type [experts, 2I, H] */
    const void* down;         /* type [experts, H, I] */
    const void* shared_gate;  /* type [shared_I, H] */
    const void* shared_up;    /* type [shared_I, H] */
    const void* shared_down;  /* type [H, shared_I] */
    const void* shared_scale; /* BF16 [1, H] (mlp.shared_expert_gate), 16-byte aligned */
    uint32_t type;            /* Q8_0 or Q4_0: routed and shared experts */
    int experts, top_k, H, I, shared_I;
} q3x_hip_moe_layer_weights;

/* Bytes of caller-owned workspace q3x_hip_moe_layer needs for `tokens`. */
size_t q3x_hip_moe_layer_workspace_bytes(const q3x_hip_moe_layer_weights* layer, int tokens);

/* The whole MoE layer for every token t (engine.cpp:406-430; CUDA moe(),
 * engine.cu:1709-1736):
 *   logits = router X[t] (BF16 matvec), top_k routing as q3x_hip_router_topk,
 *   Y[t] = sum_slot w_slot Down_e(silu(G_e X[t]) * U_e X[t])      (slot order)
 *   Y[t] += sigmoid(shared_scale . X[t]) *
 *           shared_down(silu(shared_gate X[t]) * shared_up X[t])  (added last)
 * Y is overwritten.  ids / weights ([tokens, top_k], device) receive the
 * routing when not NULL.  Requires 1 <= top_k <= min(experts, 8), experts <=
 * 1024, H, I, shared_I multiples of 32, shared_I <= I (the reference reuses
 * its 2I gate_up buffer for the shared expert, engine.cpp:100-102, 422-423),
 * X 16-byte aligned.  Replaces the routed path's caller-side router matvec,
 * shared expert and scaled add (engine.cu:1711, 1728-1735).  On return the
 * workspace begins with the router logits, FP32 [tokens, experts], that the
 * routing was computed from. */
int q3x_hip_moe_layer(const q3x_hip_moe_layer_weights* layer, const float* X, int tokens, float* Y,
                      int* ids, float* weights, void* workspace, size_t workspace_bytes,
                      hipStream_t stream);

/* dst = Q8_0/Q4_0 blocks of src[rows, cols] (FP32), the quantizers of the
 * reference's packer (scripts/pack_weights.py:299-343) applied to FP32 input:
 * Q8_0 d = max|w|/127, q = clip(copysign(floor(|w/d| + 0.5)), +-127);
 * Q4_0 d = w[argmax|w|] / -8, nibble = min(15, trunc(w/d + 8.5)); d stored as
 * fp16 round-to-nearest-even; 1/d taken in FP32.  Non-finite input is the
 * caller's responsibility (the packer rejects it; here it yields the same
 * arithmetic on IEEE specials). */
int q3x_hip_quantize(uint32_t type, const float* src, int rows, int cols, void* dst,
                     hipStream_t stream);

/* The same quantizers on BF16 src[rows, cols] (device, 16-byte aligned), the
 * packer's own input: scripts/pack_weights.py:299-343 take little-endian
 * BF16 rows and widen them to FP32 exactly (bits << 16) before quantizing,
 * so dst equals q3x_hip_quantize of the widened values bit for bit. */
int q3x_hip_quantize_bf16(uint32_t type, const uint16_t* src, int rows, int cols, void* dst,
                          hipStream_t stream);

/* A plain streaming read of bytes (16-byte aligned, a multiple of 16) of
 * device memory, as fast as this library reads HBM without any work on the
 * data: non-temporal 16-byte loads over 512 workgroups of 1024 threads.  No
 * counterpart in the reference; bench.py times it over the same weight
 * bytes as each decode matvec, so every matvec figure sits beside the read
 * rate the box reaches at that size.  *sink (4 bytes of device memory) is
 * written only on a 1-in-2^32 pattern of the data's XOR. */
int q3x_hip_read_probe(const void* buffer, size_t bytes, uint32_t* sink, hipStream_t stream);

/* ------------------------------------------------------------------------
 * model.bin -- the weight file the matmuls read (reference model_config.h,
 * engine.cpp:455-559, arch/cuda/engine.cu:2007-2188, written by
 * scripts/pack_weights.py).  A 72-byte header -- "Q3XMODL\0" and 16
 * little-endian uint32 fields (model ID, V, H, I, N, AI, AH, KVH, AD, RD, KH,
 * VH, KD, VD, CK, 262144) -- then every tensor of the model ID's fixed
 * configuration in one fixed order, each starting at the next multiple of 64
 * bytes, the file ending exactly where the last tensor ends.
 * Unlike the matmul entry points above, q3x_hip_model_load reads a file and
 * owns one device allocation until q3x_hip_model_free.
 * ------------------------------------------------------------------------ */

#define Q3X_HIP_MODEL_HEADER_BYTES 72

enum {
    Q3X_HIP_EMODEL = -4,     /* model.bin rejected; the message names why */
    Q3X_HIP_TENSOR_F32 = 3,  /* element type of the FP32 vectors (after the matrix types) */
};

/* Tensor roles, named as the reference's Model / Layer fields
 * (engine.cpp:31-64, 165-177). */
enum {
    Q3X_HIP_EMBEDDING = 0, Q3X_HIP_LM_HEAD, Q3X_HIP_FINAL_NORM,
    Q3X_HIP_INPUT_NORM, Q3X_HIP_POST_NORM,
    Q3X_HIP_DELTA_QKV, Q3X_HIP_DELTA_Z, Q3X_HIP_DELTA_A, Q3X_HIP_DELTA_B, Q3X_HIP_DELTA_CONV,
    Q3X_HIP_DELTA_ALOG, Q3X_HIP_DELTA_DT, Q3X_HIP_DELTA_NORM, Q3X_HIP_DELTA_OUT,
    Q3X_HIP_ATTN_Q, Q3X_HIP_ATTN_K, Q3X_HIP_ATTN_V, Q3X_HIP_ATTN_QNORM, Q3X_HIP_ATTN_KNORM,
    Q3X_HIP_ATTN_OUT,
    Q3X_HIP_FFN_GATE, Q3X_HIP_FFN_UP, Q3X_HIP_FFN_DOWN,
    Q3X_HIP_MOE_ROUTER, Q3X_HIP_MOE_GATE_UP, Q3X_HIP_MOE_DOWN, Q3X_HIP_MOE_SHARED_GATE,
    Q3X_HIP_MOE_SHARED_UP, Q3X_HIP_MOE_SHARED_DOWN, Q3X_HIP_MOE_SHARED_SCALE,
    Q3X_HIP_TENSOR_ROLES
};

/* One supported model (the reference's ModelConfig, model_config.h:47-57):
 * shapes, MoE sizes, the matrix type of its linear layers and whether
 * lm_head shares the embedding's storage. */
typedef struct q3x_hip_model_config {
    uint32_t id;
    const char* name;
    int V, H, I, N;
    int AI, AH, KVH, AD, RD;
    int KH, VH, KD, VD, CK;
    int experts, top_k, shared_I;
    uint32_t matrix_type;
    int tied_embeddings;
} q3x_hip_model_config;

/* One tensor of model.bin.  Matrices: [rows, cols] of `type` (an expert pool
 * is `experts` such matrices back to back); vectors: rows 1, cols elements;
 * the DeltaNet conv weight: rows DQKV, cols CK (BF16). */
typedef struct q3x_hip_tensor {
    uint32_t role;       /* Q3X_HIP_EMBEDDING ... */
    int layer;           /* 0 .. N-1, or -1 outside the layers */
    uint32_t type;       /* Q3X_HIP_MATRIX_BF16 / _Q8_0 / _Q4_0, or Q3X_HIP_TENSOR_F32 */
    int experts;         /* 0, or the number of experts of a pool */
    int rows, cols;
    uint64_t offset;     /* from the start of the file: a multiple of 64 */
    uint64_t bytes;
} q3x_hip_tensor;

/* Validates a model.bin from its first `header_bytes` (>= 72) bytes and its
 * size, with the reference loader's checks and messages (engine.cpp:481-559):
 * "bad model.bin" (shorter than the header), "wrong model.bin magic",
 * "unsupported Qwen model ID", "Qwen model.bin header mismatch" (any of the
 * 16 fields differs from the ID's configuration, model_config.h:115-141),
 * "truncated model.bin" (a tensor ends past the file), "model.bin size does
 * not match schema" (bytes left after the last tensor) -- Q3X_HIP_EMODEL with
 * *error set.  On success *config (if not NULL) receives the configuration,
 * *count the number of tensors and, when `tensors` is not NULL, tensors[0 ..
 * count) the tensors in file order (capacity < count: Q3X_HIP_EINVAL).  A
 * model with tied embeddings stores no lm_head.  Host only; reads nothing
 * past the header. */
int q3x_hip_model_layout(const void* header, size_t header_bytes, uint64_t file_size,
                         q3x_hip_model_config* config, q3x_hip_tensor* tensors, size_t capacity,
                         size_t* count, const char** error);

/* The same layout for any configuration `config` describes (the five of
 * model.bin included): the tensors in file order with their offsets (from a
 * 72-byte header, each at the next multiple of 64 bytes) and, in *bytes, the
 * size of such a file.  For weights built in memory, e.g. small synthetic
 * models.  Q3X_HIP_EINVAL for a configuration whose sizes are not positive,
 * whose heads do not divide evenly, whose quantized rows are not whole
 * 32-element blocks, or whose row counts overflow an int. */
int q3x_hip_model_schema(const q3x_hip_model_config* config, q3x_hip_tensor* tensors, size_t capacity,
                         size_t* count, uint64_t* bytes);

typedef struct q3x_hip_model q3x_hip_model;

/* Loads model.bin onto the current device (the CUDA loader, engine.cu:2032-
 * 2188): opens `path` ("cannot open model.bin"), validates it as
 * q3x_hip_model_layout before any device work, allocates one device buffer
 * of the file's size and copies the whole file into it, so that tensor t
 * lives at base + t.offset (64-byte aligned).  The copy overlaps file reads
 * and host-to-device transfers through pinned staging buffers and is
 * complete when the call returns.  Errors: Q3X_HIP_EMODEL (file rejected or
 * unreadable), Q3X_HIP_ERUNTIME ("HIP model does not fit in device memory",
 * "HIP model allocation failed", "HIP model upload failed"), Q3X_HIP_EINVAL;
 * *error names the cause.  Release with q3x_hip_model_free. */
int q3x_hip_model_load(const char* path, q3x_hip_model** model, const char** error);

/* Frees the device buffer and the handle (NULL is a no-op).  Any work that
 * reads the weights must have completed. */
void q3x_hip_model_free(q3x_hip_model* model);

/* The loaded model's configuration, tensor table (file order, owned by the
 * handle) and device buffer (base, bytes = file size).  Outputs may be NULL. */
int q3x_hip_model_info(const q3x_hip_model* model, q3x_hip_model_config* config,
                       const q3x_hip_tensor** tensors, size_t* count, const void** base,
                       uint64_t* bytes);

/* Tensor `role` of `layer` (-1 for embedding, lm_head and final_norm) and its
 * device address; a tied lm_head resolves to the embedding, as in
 * engine.cpp:500.  Q3X_HIP_EINVAL when the model has no such tensor. */
int q3x_hip_model_tensor(const q3x_hip_model* model, uint32_t role, int layer,
                         q3x_hip_tensor* tensor, const void** data);

/* The weights of MoE layer `layer` of a loaded MoE model, ready for
 * q3x_hip_moe_layer (engine.cpp:543-550: router, routed pools, shared expert
 * and its gate).  Q3X_HIP_EINVAL for a dense model or a layer out of range. */
int q3x_hip_model_moe_layer(const q3x_hip_model* model, int layer,
                            q3x_hip_moe_layer_weights* weights);

/* ------------------------------------------------------------------------
 * Decode engine: tokens through every layer of a Q8_0 / Q4_0 model on the
 * current device -- the reference's forward (engine.cpp:431-454; CUDA
 * forward and state_forward, arch/cuda/engine.cu:1961-2005, 2237-2307) over
 * this library's matmul entry points, for the backend interface
 * q3x_backend::state_* (internal.h:11-34).  The engine owns its state on the
 * device (work vectors, DeltaNet conv history and memory, KV cache, logits)
 * and a stream; one decode step is captured into a hipGraph on first use and
 * replayed for every token.  Not thread-safe: one caller per engine.
 * ------------------------------------------------------------------------ */

typedef struct q3x_hip_engine q3x_hip_engine;

enum {
    Q3X_HIP_ESTATE = -6, /* engine left failed by an earlier forward; reset or restore it */
};

/* An engine over `weights`, a device buffer laid out as q3x_hip_model_schema
 * gives for `config` (the buffer of q3x_hip_model_load qualifies), with room
 * for `context` tokens (1 .. 262144).  A forward of several tokens runs as
 * prefill chunks of `chunk` rows (0: 4096; at most `context`), whose work
 * buffers the engine holds.  Needs a Q8_0 or Q4_0 model with KD, VD <= 128,
 * AD <= 256 a multiple of 32, RD <= min(64, AD) even, 2 <= CK <= 8,
 * top_k <= 8, AH / KVH <= 8 (BF16 models: Q3X_HIP_ENOTSUP, as the matmul
 * entry points).  The weights must outlive the engine.  *error names the
 * cause of a failure. */
int q3x_hip_engine_create(const q3x_hip_model_config* config, const void* weights, int context, int chunk,
                          q3x_hip_engine** engine, const char** error);
void q3x_hip_engine_destroy(q3x_hip_engine* engine);

/* Position 0 and a zero recurrent state (state_reset, engine.cpp:158-162).
 * Also clears the failed state a forward can leave (below). */
int q3x_hip_engine_reset(q3x_hip_engine* engine);

/* tokens[0 .. count) (host) through the model at the current position, one
 * token at a time as the reference's state_forward (engine.cpp:586-589);
 * the logits of the last token when compute_logits.  Returns when done.
 * Q3X_HIP_EINVAL for a token outside [0, V) or more tokens than the context
 * has left (nothing is run).  A failure once work has been queued (a later
 * prefill chunk, the decode graph, the wait for the stream) returns its
 * code after the queued work has ended and leaves the engine failed: the
 * state may hold part of the tokens, so every forward returns
 * Q3X_HIP_ESTATE, running nothing, until q3x_hip_engine_reset or
 * q3x_hip_engine_checkpoint_restore (the reference aborts instead). */
int q3x_hip_engine_forward(q3x_hip_engine* engine, const int* tokens, int count, int compute_logits);

/* The last computed logits [V] into host memory (state_copy_logits). */
int q3x_hip_engine_logits(const q3x_hip_engine* engine, float* logits);

/* The index of the largest logit, lowest index among equals (state_argmax). */
int q3x_hip_engine_argmax(const q3x_hip_engine* engine, int* token);

/* Save / restore position, recurrent state and logits
 * (state_checkpoint_save / _restore, engine.cpp:590-604).  A restore also
 * clears the failed state. */
int q3x_hip_engine_checkpoint_save(q3x_hip_engine* engine);
int q3x_hip_engine_checkpoint_restore(q3x_hip_engine* engine);

/* Tokens processed since the last reset (-1 for NULL). */
int q3x_hip_engine_position(const q3x_hip_engine* engine);

#ifdef __cplusplus
}
#endif
#endif
