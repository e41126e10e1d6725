// hip_ops.cpp -- see hip_ops.h.
#include "hip_ops.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>

namespace qwen3x_hip {
namespace {

void check(int status, const char* what, const char* file, int line) {
    if (status == Q3X_HIP_OK) return;
    std::fprintf(stderr, "%s:%d: %s failed: %s (%d)\n", file, line, what, q3x_hip_strerror(status), status);
    std::abort();
}

#define Q3X_HIP_CHECK(call) check((call), #call, __FILE__, __LINE__)
// Fatal invariant, like Q3X_ASSERT (internal.h:76-85).
#define Q3X_HIP_ASSERT(cond) check((cond) ? Q3X_HIP_OK : Q3X_HIP_EINVAL, #cond, __FILE__, __LINE__)

}  // namespace

void mv(const Linear& linear, const float* input, float* output, hipStream_t stream) {
    Q3X_HIP_CHECK(q3x_hip_mv(linear.weight, linear.type, linear.rows, linear.columns, input, output, 0,
                             stream));
}

void mv_add(const Linear& linear, const float* input, float* output, hipStream_t stream) {
    Q3X_HIP_CHECK(q3x_hip_mv(linear.weight, linear.type, linear.rows, linear.columns, input, output, 1,
                             stream));
}

void projections(const Linear* linears, float* const* outputs, int count, const float* input,
                 hipStream_t stream) {
    Q3X_HIP_ASSERT(count >= 1 && count <= Q3X_HIP_MV_MULTI_MAX);
    q3x_hip_mv_item items[Q3X_HIP_MV_MULTI_MAX];
    for (int i = 0; i < count; ++i) {
        Q3X_HIP_ASSERT(linears[i].type == linears[0].type && linears[i].columns == linears[0].columns);
        items[i] = q3x_hip_mv_item{linears[i].weight, linears[i].rows, outputs[i], 0};
    }
    Q3X_HIP_CHECK(q3x_hip_mv_multi(items, count, linears[0].type, linears[0].columns, input, stream));
}

void batch_mv(const Linear& linear, const float* input, float* output, int count, bool add,
              hipStream_t stream) {
    Q3X_HIP_CHECK(q3x_hip_gemm(linear.weight, linear.type, linear.rows, linear.columns, input, count,
                               output, add ? 1 : 0, stream));
}

size_t batch_mv_workspace_bytes(const Linear& linear, int count) {
    return q3x_hip_gemm_workspace_bytes(linear.type, linear.rows, linear.columns, count);
}

void batch_mv(const Linear& linear, const float* input, float* output, int count, bool add, void* workspace,
              size_t workspace_bytes, hipStream_t stream) {
    Q3X_HIP_CHECK(q3x_hip_gemm_ws(linear.weight, linear.type, linear.rows, linear.columns, input, count, output,
                                  add ? 1 : 0, workspace, workspace_bytes, stream));
}

void embed(const Linear& table, int token, float* output, hipStream_t stream) {
    if (token < 0 || token >= table.rows) {
        std::fprintf(stderr, "embedding token=%d rows=%d\n", token, table.rows);
        std::abort();
    }
    Q3X_HIP_CHECK(q3x_hip_dequant(table.weight, table.type, table.columns, token, 1, output, stream));
}

void router_top_k(const float* logits, int tokens, int experts, int top_k, int* ids, float* weights,
                  hipStream_t stream) {
    Q3X_HIP_CHECK(q3x_hip_router_topk(logits, tokens, experts, top_k, ids, weights, stream));
}

size_t moe_workspace_bytes(int tokens, int experts, int top_k, int H, int I) {
    return q3x_hip_moe_workspace_bytes(tokens, experts, top_k, H, I);
}

void moe_routed(const ExpertLinear& gate_up, const ExpertLinear& down, const float* input, int tokens,
                const int* ids, const float* weights, int top_k, float* output, bool add, void* workspace,
                size_t workspace_bytes, hipStream_t stream) {
    if (gate_up.type != down.type || gate_up.experts != down.experts || gate_up.columns != down.rows ||
        gate_up.rows != 2 * down.columns) {
        std::fprintf(stderr, "moe_routed: gate_up [%d,%d,%d] and down [%d,%d,%d] do not match\n",
                     gate_up.experts, gate_up.rows, gate_up.columns, down.experts, down.rows, down.columns);
        std::abort();
    }
    Q3X_HIP_CHECK(q3x_hip_moe_routed(gate_up.weight, down.weight, gate_up.type, gate_up.experts,
                                     gate_up.columns, down.columns, input, tokens, ids, weights, top_k,
                                     output, add ? 1 : 0, workspace, workspace_bytes, stream));
}

namespace {

q3x_hip_moe_layer_weights layer_of(const MoeWeights& w, int top_k) {
    const bool ok = w.router.type == MATRIX_BF16 && w.shared_scale.type == MATRIX_BF16 &&
                    w.gate_up.type == w.down.type && w.shared_gate.type == w.gate_up.type &&
                    w.shared_up.type == w.gate_up.type && w.shared_down.type == w.gate_up.type &&
                    w.router.rows == w.gate_up.experts && w.router.columns == w.gate_up.columns &&
                    w.down.experts == w.gate_up.experts && w.down.rows == w.gate_up.columns &&
                    w.gate_up.rows == 2 * w.down.columns && w.shared_gate.columns == w.gate_up.columns &&
                    w.shared_up.rows == w.shared_gate.rows && w.shared_up.columns == w.gate_up.columns &&
                    w.shared_down.rows == w.gate_up.columns && w.shared_down.columns == w.shared_gate.rows &&
                    w.shared_scale.rows == 1 && w.shared_scale.columns == w.gate_up.columns;
    if (!ok) {
        std::fprintf(stderr, "moe: the layer's matrices do not match (engine.cu:97-101 shapes)\n");
        std::abort();
    }
    return q3x_hip_moe_layer_weights{w.router.weight, w.gate_up.weight, w.down.weight, w.shared_gate.weight,
                                     w.shared_up.weight, w.shared_down.weight, w.shared_scale.weight,
                                     w.gate_up.type, w.gate_up.experts, top_k, w.gate_up.columns,
                                     w.down.columns, w.shared_gate.rows};
}

}  // namespace

size_t moe_workspace_bytes(const MoeWeights& weights, int top_k, int tokens) {
    const q3x_hip_moe_layer_weights layer = layer_of(weights, top_k);
    return q3x_hip_moe_layer_workspace_bytes(&layer, tokens);
}

void moe(const MoeWeights& weights, const float* input, int tokens, float* output, int top_k, int* ids,
         float* routing_weights, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const q3x_hip_moe_layer_weights layer = layer_of(weights, top_k);
    Q3X_HIP_CHECK(q3x_hip_moe_layer(&layer, input, tokens, output, ids, routing_weights, workspace,
                                    workspace_bytes, stream));
}

Model::~Model() {
    delete[] layers;
    q3x_hip_model_free(handle);
}

bool Model::load(const char* path, const char** error) {
    q3x_hip_model* loaded = nullptr;
    const char* message = nullptr;
    if (q3x_hip_model_load(path, &loaded, &message) != Q3X_HIP_OK) {
        *error = message ? message : "cannot load model.bin";
        return false;
    }
    const q3x_hip_tensor* table = nullptr;
    size_t count = 0;
    const void* base = nullptr;
    q3x_hip_model_config c{};
    Q3X_HIP_CHECK(q3x_hip_model_info(loaded, &c, &table, &count, &base, nullptr));
    Layer* bound = new Layer[c.N];
    for (size_t i = 0; i < count; ++i) {
        const q3x_hip_tensor& t = table[i];
        const void* p = static_cast<const uint8_t*>(base) + t.offset;
        const Linear linear{p, t.rows, t.cols, static_cast<MatrixType>(t.type)};
        const ExpertLinear pool{p, t.experts, t.rows, t.cols, static_cast<MatrixType>(t.type)};
        const uint16_t* bf16 = static_cast<const uint16_t*>(p);
        const float* f32 = static_cast<const float*>(p);
        if (t.layer < 0) {
            if (t.role == Q3X_HIP_EMBEDDING) embedding = linear;
            else if (t.role == Q3X_HIP_LM_HEAD) lm_head = linear;
            else if (t.role == Q3X_HIP_FINAL_NORM) final_norm = bf16;
            continue;
        }
        Layer& l = bound[t.layer];
        switch (t.role) {
        case Q3X_HIP_INPUT_NORM: l.input_norm = bf16; break;
        case Q3X_HIP_POST_NORM: l.post_norm = bf16; break;
        case Q3X_HIP_DELTA_QKV: l.delta.qkv = linear; break;
        case Q3X_HIP_DELTA_Z: l.delta.z = linear; break;
        case Q3X_HIP_DELTA_A: l.delta.a = linear; break;
        case Q3X_HIP_DELTA_B: l.delta.b = linear; break;
        case Q3X_HIP_DELTA_CONV: l.delta.conv = bf16; break;
        case Q3X_HIP_DELTA_ALOG: l.delta.alog = f32; break;
        case Q3X_HIP_DELTA_DT: l.delta.dt = bf16; break;
        case Q3X_HIP_DELTA_NORM: l.delta.norm = f32; break;
        case Q3X_HIP_DELTA_OUT: l.delta.out = linear; break;
        case Q3X_HIP_ATTN_Q: l.attention.q = linear; break;
        case Q3X_HIP_ATTN_K: l.attention.k = linear; break;
        case Q3X_HIP_ATTN_V: l.attention.v = linear; break;
        case Q3X_HIP_ATTN_QNORM: l.attention.qnorm = bf16; break;
        case Q3X_HIP_ATTN_KNORM: l.attention.knorm = bf16; break;
        case Q3X_HIP_ATTN_OUT: l.attention.out = linear; break;
        case Q3X_HIP_FFN_GATE: l.gate = linear; break;
        case Q3X_HIP_FFN_UP: l.up = linear; break;
        case Q3X_HIP_FFN_DOWN: l.down = linear; break;
        case Q3X_HIP_MOE_ROUTER: l.moe.router = linear; break;
        case Q3X_HIP_MOE_GATE_UP: l.moe.gate_up = pool; break;
        case Q3X_HIP_MOE_DOWN: l.moe.down = pool; break;
        case Q3X_HIP_MOE_SHARED_GATE: l.moe.shared_gate = linear; break;
        case Q3X_HIP_MOE_SHARED_UP: l.moe.shared_up = linear; break;
        case Q3X_HIP_MOE_SHARED_DOWN: l.moe.shared_down = linear; break;
        case Q3X_HIP_MOE_SHARED_SCALE: l.moe.shared_scale = linear; break;
        default: Q3X_HIP_ASSERT(false);
        }
    }
    if (c.tied_embeddings) lm_head = embedding;  // engine.cpp:500
    delete[] layers;
    q3x_hip_model_free(handle);
    config = c;
    layers = bound;
    handle = loaded;
    *error = nullptr;
    return true;
}

}  // namespace qwen3x_hip
