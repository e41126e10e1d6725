// ref_shim.cpp -- C entry points into the reference CPU engine, compiled from
// the reference sources where they lie (TEST INFRASTRUCTURE ONLY).
//
// Like the reference's own tests (tests/q8_cpu_test.cpp:11,
// tests/q4_cpu_test.cpp), this file includes engine.cpp to reach its
// internal functions, and exports them with plain C signatures so the parity
// tests can compare this repository's oracle against the reference bit for bit.
// Built by `make -C oracle ref` into oracle/_ref/ (git-ignored).
#include "engine.cpp"
#include "q4.h"

#include <vector>

extern "C" {

int q3xr_quantized_bytes(uint32_t type, int rows, int cols, size_t* bytes) {
    return q3x_cpu::quantized_bytes(static_cast<q3x_model::MatrixType>(type), rows, cols,
                                    bytes) ? 1 : 0;
}

// arch/cpu.cpp:181-190
int q3xr_try_embed(const void* weights, uint32_t type, int cols, int row, float* out) {
    if (type > q3x_model::MATRIX_Q4_0) return 0;
    return q3x_cpu::try_embed(weights, static_cast<q3x_model::MatrixType>(type), cols, row,
                              out) ? 1 : 0;
}

// arch/cpu.cpp:192-226 (serial on x86)
int q3xr_try_mv(const void* weights, uint32_t type, int rows, int cols, const float* x,
                float* y) {
    if (type > q3x_model::MATRIX_Q4_0) return 0;
    return q3x_cpu::try_mv(weights, static_cast<q3x_model::MatrixType>(type), rows, cols, x,
                           y) ? 1 : 0;
}

// engine.cpp:377-405 (probabilities[ids[slot]] holds the renormalised weight)
void q3xr_router_top_k(const float* logits, int experts, int top_k, int* ids,
                       float* probabilities) {
    q3x_backend::router_top_k(logits, experts, top_k, ids, probabilities);
}

float q3xr_sigmoid(float x) { return q3x_backend::sigmoid(x); }
float q3xr_silu(float x) { return q3x_backend::silu(x); }

// engine.cpp:406-430 for one token: BF16 router [E, H], Q4_0 experts
// gate_up [E, 2I, H] and down [E, H, I].  The shared expert is given all-zero
// Q4_0 blocks (scale 0) so it adds exactly zero; `logits` receives the router
// output the reference computed, `ids` the selected experts.
void q3xr_moe_q4(const uint16_t* router, const void* gate_up, const void* down,
                 int experts, int H, int I, int top_k, const float* input,
                 float* logits, int* ids, float* out) {
    // Work (engine.cpp:84-110) sizes delta_output, which moe() reuses for the
    // expert down output of H floats, as VH * VD: take VD = H.
    const q3x_model::ModelConfig config {
        1, "synthetic-MoE", 64, H, I, 1,
        1, 1, 1, 32, 16, 1, 1, 32, H, 4,
        experts, top_k, 32, q3x_model::MATRIX_Q4_0, false,
    };
    const int shared_I = 32;
    std::vector<q3x_q4::Block> shared_gate(static_cast<size_t>(shared_I) * H / 32);
    std::vector<q3x_q4::Block> shared_up(shared_gate.size());
    std::vector<q3x_q4::Block> shared_down(static_cast<size_t>(H) * shared_I / 32);
    std::vector<uint16_t> shared_scale(H, 0);
    for (auto* pool : {&shared_gate, &shared_up, &shared_down})
        for (auto& block : *pool) { block.scale = 0; std::memset(block.values, 0x88, 16); }
    q3x_backend::MoeWeights weights {
        {router, experts, H, q3x_model::MATRIX_BF16},
        {gate_up, experts, 2 * I, H, q3x_model::MATRIX_Q4_0},
        {down, experts, H, I, q3x_model::MATRIX_Q4_0},
        {shared_gate.data(), shared_I, H, q3x_model::MATRIX_Q4_0},
        {shared_up.data(), shared_I, H, q3x_model::MATRIX_Q4_0},
        {shared_down.data(), H, shared_I, q3x_model::MATRIX_Q4_0},
        {shared_scale.data(), 1, H, q3x_model::MATRIX_BF16},
    };
    q3x_backend::Work work(config);
    q3x_backend::mv(weights.router, input, logits);
    q3x_backend::moe(weights, input, work, out, config);
    for (int slot = 0; slot < top_k; ++slot) ids[slot] = work.expert_ids[slot];
}


// The routed loop of moe() (engine.cpp:411-420) for one token with the
// selection given: out = 0, then per slot expert_mv of gate_up, silu(gate) *
// up, expert_mv of down and out += weight * down, with the reference's own
// expert_mv and silu.  For the CPU baseline of the routed-expert benchmark.
void q3xr_moe_routed(uint32_t type, const void* gate_up, const void* down, int experts, int H, int I,
                     const float* input, const int* ids, const float* weights, int top_k, float* out) {
    const auto t = static_cast<q3x_model::MatrixType>(type);
    const q3x_backend::ExpertLinear gu {gate_up, experts, 2 * I, H, t};
    const q3x_backend::ExpertLinear dn {down, experts, H, I, t};
    std::vector<float> gate_up_out(2 * static_cast<size_t>(I)), h(I), d(H);
    std::fill(out, out + H, 0.0f);
    for (int slot = 0; slot < top_k; ++slot) {
        q3x_backend::expert_mv(gu, ids[slot], input, gate_up_out.data());
        for (int i = 0; i < I; ++i) h[i] = q3x_backend::silu(gate_up_out[i]) * gate_up_out[I + i];
        q3x_backend::expert_mv(dn, ids[slot], h.data(), d.data());
        for (int i = 0; i < H; ++i) out[i] += weights[slot] * d[i];
    }
}
// engine.cpp:207-212, the BF16 branch of mv().
void q3xr_mv_bf16(const uint16_t* weights, int rows, int cols, const float* x, float* y) {
    q3x_backend::mv({weights, rows, cols, q3x_model::MATRIX_BF16}, x, y);
}

// engine.cpp:406-430 for one token with every weight given: BF16 router
// [E, H] and shared_scale [1, H]; experts gate_up [E, 2I, H], down [E, H, I]
// and the shared expert (gate/up [shared_I, H], down [H, shared_I]) of
// `type`.  shared_I <= I (moe() writes the shared up output at
// ffn_gate_up + I).  `ids` receives the selected experts.
void q3xr_moe_layer(uint32_t type, const uint16_t* router, const void* gate_up, const void* down,
                    const void* shared_gate, const void* shared_up, const void* shared_down,
                    const uint16_t* shared_scale, int experts, int H, int I, int shared_I, int top_k,
                    const float* input, float* out, int* ids) {
    const auto t = static_cast<q3x_model::MatrixType>(type);
    // Work (engine.cpp:84-110) sizes delta_output, which moe() reuses for the
    // down outputs of H floats, as VH * VD: take VD = H.
    const q3x_model::ModelConfig config {
        1, "synthetic-MoE", 64, H, I, 1,
        1, 1, 1, 32, 16, 1, 1, 32, H, 4,
        experts, top_k, shared_I, t, false,
    };
    q3x_backend::MoeWeights weights {
        {router, experts, H, q3x_model::MATRIX_BF16},
        {gate_up, experts, 2 * I, H, t},
        {down, experts, H, I, t},
        {shared_gate, shared_I, H, t},
        {shared_up, shared_I, H, t},
        {shared_down, H, shared_I, t},
        {shared_scale, 1, H, q3x_model::MATRIX_BF16},
    };
    q3x_backend::Work work(config);
    q3x_backend::moe(weights, input, work, out, config);
    for (int slot = 0; slot < top_k; ++slot) ids[slot] = work.expert_ids[slot];
}
// engine.cpp:481-559: the reference's own loader on the file at `path` (it
// maps the file and reads nothing past the header).  On success returns 1 and
// lists every tensor it bound, in file order: the offset from the start of
// the file and (rows, cols, experts, type), with -1 for the fields a bare
// vector pointer lacks.  On failure returns 0 with the reference's message.
int q3xr_model_load(const char* path, uint64_t* offsets, int* shapes, size_t capacity, size_t* count,
                    const char** error) {
    q3x_backend::Model model;
    const char* message = nullptr;
    *count = 0;
    if (!model.load(path, &message)) {
        *error = message;
        return 0;
    }
    size_t n = 0;
    auto put = [&](const void* p, int rows, int cols, int experts, int type) {
        if (n < capacity) {
            offsets[n] = static_cast<uint64_t>(static_cast<const uint8_t*>(p) - model.file);
            int* s = shapes + 4 * n;
            s[0] = rows; s[1] = cols; s[2] = experts; s[3] = type;
        }
        ++n;
    };
    auto linear = [&](const q3x_backend::Linear& l) { put(l.w, l.rows, l.cols, 0, l.type); };
    auto pool = [&](const q3x_backend::ExpertLinear& e) { put(e.w, e.rows, e.cols, e.experts, e.type); };
    auto vec = [&](const void* p) { put(p, -1, -1, -1, -1); };
    const auto& c = *model.config;
    linear(model.embedding);
    if (!c.tied_embeddings) linear(model.lm_head);
    vec(model.final_norm);
    for (int i = 0; i < c.N; ++i) {
        const q3x_backend::Layer& l = model.layer[i];
        vec(l.input_norm);
        if (i % c.AI != c.AI - 1) {
            linear(l.delta.qkv); linear(l.delta.z); linear(l.delta.a); linear(l.delta.b);
            vec(l.delta.conv); vec(l.delta.alog); vec(l.delta.dt); vec(l.delta.norm);
            linear(l.delta.out);
        } else {
            linear(l.attention.q); linear(l.attention.k); linear(l.attention.v);
            vec(l.attention.qnorm); vec(l.attention.knorm);
            linear(l.attention.out);
        }
        vec(l.post_norm);
        if (c.experts) {
            linear(l.moe.router); pool(l.moe.gate_up); pool(l.moe.down);
            linear(l.moe.shared_gate); linear(l.moe.shared_up); linear(l.moe.shared_down);
            linear(l.moe.shared_scale);
        } else {
            linear(l.gate); linear(l.up); linear(l.down);
        }
    }
    *count = n;
    return 1;
}
// engine.cpp:431-454 forward, token by token, on a model given in memory:
// `cfg` holds the ModelConfig fields (id, V, H, I, N, AI, AH, KVH, AD, RD, KH,
// VH, KD, VD, CK, experts, top_k, shared_I, matrix_type, tied_embeddings),
// `image` the weights laid out as model.bin, and (role, layer, offset) each
// tensor's place in it, roles numbered as the HIP library's tensor roles.
// logits[t * V ..] receives the logits after token t.  Returns 0 when the
// configuration cannot be built.
int q3xr_forward(const int* cfg, const uint8_t* image, const int* roles, const int* layers,
                 const uint64_t* offsets, int tensors, const int* tokens, int count, float* logits) {
    const q3x_model::ModelConfig config {
        static_cast<uint32_t>(cfg[0]), "synthetic", cfg[1], cfg[2], cfg[3], cfg[4],
        cfg[5], cfg[6], cfg[7], cfg[8], cfg[9], cfg[10], cfg[11], cfg[12], cfg[13], cfg[14],
        cfg[15], cfg[16], cfg[17], static_cast<q3x_model::MatrixType>(cfg[18]), cfg[19] != 0,
    };
    const auto& c = config;
    const auto M = c.matrix_type;
    const auto BF = q3x_model::MATRIX_BF16;
    const int AS = c.AH * c.AD, KVW = c.KVH * c.AD, DO = c.VH * c.VD, DQKV = 2 * c.KH * c.KD + DO;
    q3x_backend::Model model;
    model.config = &config;
    model.layer.reset(new q3x_backend::Layer[c.N]);
    for (int i = 0; i < tensors; ++i) {
        const void* p = image + offsets[i];
        const auto* bf = static_cast<const q3x_backend::BF16*>(p);
        const auto* f32 = static_cast<const float*>(p);
        const int l = layers[i];
        auto lin = [&](int rows, int cols, q3x_model::MatrixType t) { return q3x_backend::Linear{p, rows, cols, t}; };
        switch (roles[i]) {
        case 0: model.embedding = lin(c.V, c.H, M); break;
        case 1: model.lm_head = lin(c.V, c.H, M); break;
        case 2: model.final_norm = bf; break;
        case 3: model.layer[l].input_norm = bf; break;
        case 4: model.layer[l].post_norm = bf; break;
        case 5: model.layer[l].delta.qkv = lin(DQKV, c.H, M); break;
        case 6: model.layer[l].delta.z = lin(DO, c.H, M); break;
        case 7: model.layer[l].delta.a = lin(c.VH, c.H, M); break;
        case 8: model.layer[l].delta.b = lin(c.VH, c.H, M); break;
        case 9: model.layer[l].delta.conv = bf; break;
        case 10: model.layer[l].delta.alog = f32; break;
        case 11: model.layer[l].delta.dt = bf; break;
        case 12: model.layer[l].delta.norm = f32; break;
        case 13: model.layer[l].delta.out = lin(c.H, DO, M); break;
        case 14: model.layer[l].attention.q = lin(2 * AS, c.H, M); break;
        case 15: model.layer[l].attention.k = lin(KVW, c.H, M); break;
        case 16: model.layer[l].attention.v = lin(KVW, c.H, M); break;
        case 17: model.layer[l].attention.qnorm = bf; break;
        case 18: model.layer[l].attention.knorm = bf; break;
        case 19: model.layer[l].attention.out = lin(c.H, AS, M); break;
        case 20: model.layer[l].gate = lin(c.I, c.H, M); break;
        case 21: model.layer[l].up = lin(c.I, c.H, M); break;
        case 22: model.layer[l].down = lin(c.H, c.I, M); break;
        case 23: model.layer[l].moe.router = lin(c.experts, c.H, BF); break;
        case 24: model.layer[l].moe.gate_up = {p, c.experts, 2 * c.I, c.H, M}; break;
        case 25: model.layer[l].moe.down = {p, c.experts, c.H, c.I, M}; break;
        case 26: model.layer[l].moe.shared_gate = lin(c.shared_I, c.H, M); break;
        case 27: model.layer[l].moe.shared_up = lin(c.shared_I, c.H, M); break;
        case 28: model.layer[l].moe.shared_down = lin(c.H, c.shared_I, M); break;
        case 29: model.layer[l].moe.shared_scale = lin(1, c.H, BF); break;
        default: return 0;
        }
    }
    if (c.tied_embeddings) model.lm_head = model.embedding;
    q3x_backend::State state(config, count);
    for (int t = 0; t < count; ++t) {
        q3x_backend::forward(model, state, tokens[t], true);
        std::memcpy(logits + static_cast<size_t>(t) * c.V, state.work.logits, sizeof(float) * c.V);
    }
    return 1;
}
}  // extern "C"
