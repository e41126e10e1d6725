// hip_ops.cpp -- see hip_ops.h.
#include "hip_ops.h"

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

}  // namespace qwen3x_hip
