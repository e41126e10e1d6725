// hip_ops.h -- C++ host interface of the HIP backend's quantized matmul, in
// the shape of the reference CUDA backend's host helpers so an arch/hip
// engine can call it exactly where engine.cu calls mv / mv_add / batch_mv /
// moe (the routed part, or the whole layer).  Every function enqueues on `stream` and, like the reference (CUDA_OK
// and Q3X_ASSERT, arch/cuda/engine.cu:48-56, internal.h:76-85), reports and
// aborts on any error.  The work itself is done by the C ABI in q3x_hip.h.
#pragma once

#include <cstddef>
#include <cstdint>

#include "q3x_hip.h"

namespace qwen3x_hip {

// q3x_model::MatrixType (model_config.h:16-20).
enum MatrixType : uint32_t {
    MATRIX_BF16 = Q3X_HIP_MATRIX_BF16,
    MATRIX_Q8_0 = Q3X_HIP_MATRIX_Q8_0,
    MATRIX_Q4_0 = Q3X_HIP_MATRIX_Q4_0,
};

// engine.cu:68-73
struct Linear {
    const void* weight = nullptr;
    int rows = 0;
    int columns = 0;
    MatrixType type = MATRIX_BF16;
};

// engine.cu:89-95: experts contiguous matrices W[experts, rows, columns].
struct ExpertLinear {
    const void* weight = nullptr;
    int experts = 0;
    int rows = 0;
    int columns = 0;
    MatrixType type = MATRIX_BF16;
};

// output[rows] = W input (engine.cu:1531).
void mv(const Linear& linear, const float* input, float* output, hipStream_t stream);
// output[rows] += W input (engine.cu:1547).
void mv_add(const Linear& linear, const float* input, float* output, hipStream_t stream);
// outputs[i] = linears[i] input for count (1..8) matrices of one type and
// width in one launch: the projection helpers attention_projections (q, k,
// v), ffn_projections (gate, up) and delta_projections (qkv, z, a, b)
// (engine.cu:1599-1661).
void projections(const Linear* linears, float* const* outputs, int count, const float* input,
                 hipStream_t stream);
// output[count, rows] (+)= input[count, columns] W^T (engine.cu:1568, without
// the cuBLAS handle and BF16 staging buffer of the BF16 path).
void batch_mv(const Linear& linear, const float* input, float* output, int count, bool add,
              hipStream_t stream);
// The same with a caller-owned workspace of at least
// batch_mv_workspace_bytes(linear, count) bytes: shapes of few output tiles
// over a long K split K over workgroups (deterministic; another sum order).
size_t batch_mv_workspace_bytes(const Linear& linear, int count);
void batch_mv(const Linear& linear, const float* input, float* output, int count, bool add, void* workspace,
              size_t workspace_bytes, hipStream_t stream);
// output[columns] = dequantised row `token` (engine.cu:1499 embed).
void embed(const Linear& table, int token, float* output, hipStream_t stream);
// ids / weights [tokens, top_k] from logits [tokens, experts] (engine.cu:1153).
void router_top_k(const float* logits, int tokens, int experts, int top_k, int* ids, float* weights,
                  hipStream_t stream);
// Routed experts of `tokens` tokens (engine.cu:1709-1726 routed part):
// output (+)= sum_slot weights * down_e(silu(gate_e x) * up_e x).
size_t moe_workspace_bytes(int tokens, int experts, int top_k, int H, int I);
void moe_routed(const ExpertLinear& gate_up, const ExpertLinear& down, const float* input, int tokens,
                const int* ids, const float* weights, int top_k, float* output, bool add, void* workspace,
                size_t workspace_bytes, hipStream_t stream);

// engine.cu:97-101: router BF16 [experts, H]; routed experts; shared expert
// gate / up [shared_I, H], down [H, shared_I]; shared_scale BF16 [1, H].
struct MoeWeights {
    Linear router;
    ExpertLinear gate_up, down;
    Linear shared_gate, shared_up, shared_down, shared_scale;
};

// The whole MoE layer of `tokens` tokens (engine.cu:1709-1736 moe()):
// output = routed experts + sigmoid(shared_scale x) * shared expert(x).
// ids / weights ([tokens, top_k], device) receive the routing when not null.
size_t moe_workspace_bytes(const MoeWeights& weights, int top_k, int tokens);
void moe(const MoeWeights& weights, const float* input, int tokens, float* output, int top_k, int* ids,
         float* routing_weights, void* workspace, size_t workspace_bytes, hipStream_t stream);

// The rest of a layer's weights as model.bin stores them (engine.cpp:37-64):
// DeltaNet and attention projections, norms, and the dense FFN.  BF16
// vectors are uint16 device pointers, FP32 vectors float device pointers.
struct DeltaWeights {
    Linear qkv, z, a, b, out;
    const uint16_t* conv = nullptr;  // [DQKV, CK]
    const float* alog = nullptr;     // [VH]
    const uint16_t* dt = nullptr;    // [VH]
    const float* norm = nullptr;     // [VD]
};
struct AttentionWeights {
    Linear q, k, v, out;
    const uint16_t *qnorm = nullptr, *knorm = nullptr;  // [AD]
};
struct Layer {
    const uint16_t *input_norm = nullptr, *post_norm = nullptr;  // [H]
    Linear gate, up, down;  // dense models
    MoeWeights moe;         // MoE models
    DeltaWeights delta;     // layers with i % AI != AI - 1
    AttentionWeights attention;
};

// model.bin on the current device (the reference's CUDA Model::load,
// engine.cu:2032-2188): one device buffer holding the whole file, every
// field a device pointer into it.  load() returns false with the loader's
// message (engine.cpp:481-559 messages) and leaves the model empty.
struct Model {
    q3x_hip_model_config config{};
    Linear embedding, lm_head;  // lm_head == embedding for tied models
    const uint16_t* final_norm = nullptr;
    Layer* layers = nullptr;    // config.N layers
    q3x_hip_model* handle = nullptr;

    Model() = default;
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;
    ~Model();
    bool load(const char* path, const char** error);
};

}  // namespace qwen3x_hip
