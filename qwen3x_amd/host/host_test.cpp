// host_test.cpp -- the reference's GPU/CPU quantized-path unit tests, restated
// against the HIP backend through the C++ host interface (hip_ops.h).
//
// Cases and tolerances follow tests/q4_cuda_test.cu (q4_mv_test :31-60,
// router_test :109-131, expert_moe_test :62-107), tests/q8_cpu_test.cpp
// (fixed 2x64 Q8_0 vector and embed, :271-318; plus the projection helper of
// engine.cu:1607-1619 on the same matrix) and tests/q4_cpu_test.cpp
// (q4_math_test :138-178, moe_test :217-276 -- the whole MoE layer), and the
// loader tests on sparse full-size model.bin files (q8_cpu_test.cpp:222-264,
// q4_cpu_test.cpp:85-136) against the device loader.  Exit 0 = pass, 77 = no
// GPU (the reference CI's skip code, .github/workflows/ci.yml:53-55), anything
// else = failure.
#include <fcntl.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include <hip/hip_runtime.h>

#include "backend.h"
#include "hip_ops.h"

namespace {

#define HIP_OK(call)                                                                    \
    do {                                                                                \
        const hipError_t e = (call);                                                    \
        if (e != hipSuccess) {                                                          \
            std::fprintf(stderr, "%s:%d: %s: %s\n", __FILE__, __LINE__, #call,         \
                         hipGetErrorString(e));                                         \
            std::exit(1);                                                               \
        }                                                                               \
    } while (0)

#define CHECK(cond)                                                                     \
    do {                                                                                \
        if (!(cond)) {                                                                  \
            std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
            std::exit(1);                                                               \
        }                                                                               \
    } while (0)

struct Q8Block { uint16_t scale; int8_t values[32]; };
struct Q4Block { uint16_t scale; uint8_t values[16]; };
static_assert(sizeof(Q8Block) == 34, "Q8_0 block layout");
static_assert(sizeof(Q4Block) == 18, "Q4_0 block layout");

template <typename T>
T* device_copy(const T* source, size_t count) {
    T* result = nullptr;
    HIP_OK(hipMalloc(&result, count * sizeof(T)));
    HIP_OK(hipMemcpy(result, source, count * sizeof(T), hipMemcpyHostToDevice));
    return result;
}

template <typename T>
std::vector<T> host_copy(const T* source, size_t count) {
    std::vector<T> out(count);
    HIP_OK(hipMemcpy(out.data(), source, count * sizeof(T), hipMemcpyDeviceToHost));
    return out;
}

float* device_floats(size_t count) {
    float* p = nullptr;
    HIP_OK(hipMalloc(&p, count * sizeof(float)));
    HIP_OK(hipMemset(p, 0, count * sizeof(float)));
    return p;
}

float silu(float x) {  // engine.cpp:187-191
    const float s = x >= 0.0f ? 1.0f / (1.0f + std::exp(-x)) : std::exp(x) / (1.0f + std::exp(x));
    return x * s;
}

// tests/q4_cuda_test.cu:31-60
void q4_mv_test() {
    Q4Block host[2]{};
    host[0].scale = 0x3c00;
    host[1].scale = 0x3800;
    for (int i = 0; i < 16; ++i) {
        host[0].values[i] = static_cast<uint8_t>(i | ((15 - i) << 4));
        host[1].values[i] = static_cast<uint8_t>((15 - i) | (i << 4));
    }
    float input[32];
    for (int i = 0; i < 32; ++i) input[i] = (i % 9 - 4) * 0.25f;
    float expected[2]{};
    for (int row = 0; row < 2; ++row) {
        const float scale = row == 0 ? 1.0f : 0.5f;
        for (int i = 0; i < 16; ++i) {
            expected[row] += scale * ((host[row].values[i] & 15) - 8) * input[i];
            expected[row] += scale * ((host[row].values[i] >> 4) - 8) * input[i + 16];
        }
    }
    auto* weight = device_copy(host, 2);
    auto* device_input = device_copy(input, 32);
    float* device_output = device_floats(2);
    qwen3x_hip::mv({weight, 2, 32, qwen3x_hip::MATRIX_Q4_0}, device_input, device_output, nullptr);
    const auto output = host_copy(device_output, 2);
    CHECK(std::abs(output[0] - expected[0]) < 1e-5f);
    CHECK(std::abs(output[1] - expected[1]) < 1e-5f);
    // mv_add accumulates on top.
    qwen3x_hip::mv_add({weight, 2, 32, qwen3x_hip::MATRIX_Q4_0}, device_input, device_output, nullptr);
    const auto twice = host_copy(device_output, 2);
    CHECK(std::abs(twice[0] - 2 * expected[0]) < 2e-5f);
    CHECK(std::abs(twice[1] - 2 * expected[1]) < 2e-5f);
    HIP_OK(hipFree(weight)); HIP_OK(hipFree(device_input)); HIP_OK(hipFree(device_output));
}

// tests/q8_cpu_test.cpp:271-318 (main): fixed 2x64 Q8_0, then embed row 1.
void q8_fixed_test() {
    Q8Block blocks[4]{};
    const uint16_t scales[4] = {0x3c00, 0x3800, 0x4000, 0x3400};
    for (int block = 0; block < 4; ++block) {
        blocks[block].scale = scales[block];
        for (int index = 0; index < 32; ++index)
            blocks[block].values[index] = static_cast<int8_t>((index % 9) - 4 + block);
    }
    float input[64];
    for (int index = 0; index < 64; ++index) input[index] = (index % 7 - 3) * 0.125f;
    const float decoded_scales[4] = {1.0f, 0.5f, 2.0f, 0.25f};
    float expected[2]{};
    for (int row = 0; row < 2; ++row)
        for (int block = 0; block < 2; ++block) {
            float inner = 0.0f;
            for (int index = 0; index < 32; ++index)
                inner += blocks[row * 2 + block].values[index] * input[block * 32 + index];
            expected[row] += decoded_scales[row * 2 + block] * inner;
        }
    auto* weight = device_copy(blocks, 4);
    auto* device_input = device_copy(input, 64);
    float* device_output = device_floats(2);
    const qwen3x_hip::Linear matrix{weight, 2, 64, qwen3x_hip::MATRIX_Q8_0};
    qwen3x_hip::mv(matrix, device_input, device_output, nullptr);
    const auto output = host_copy(device_output, 2);
    CHECK(std::abs(output[0] - expected[0]) < 1e-6f);
    CHECK(std::abs(output[1] - expected[1]) < 1e-6f);

    float* device_embedding = device_floats(64);
    qwen3x_hip::embed(matrix, 1, device_embedding, nullptr);
    const auto embedding = host_copy(device_embedding, 64);
    for (int block = 0; block < 2; ++block)
        for (int index = 0; index < 32; ++index)
            CHECK(embedding[block * 32 + index] == decoded_scales[2 + block] * blocks[2 + block].values[index]);

    // projections: the same matrix twice plus its first row alone, one launch,
    // equal to mv bit for bit.
    {
        float* outs[3] = {device_floats(2), device_floats(2), device_floats(1)};
        const qwen3x_hip::Linear linears[3] = {matrix, matrix, {weight, 1, 64, qwen3x_hip::MATRIX_Q8_0}};
        qwen3x_hip::projections(linears, outs, 3, device_input, nullptr);
        for (int i = 0; i < 3; ++i) {
            const auto got = host_copy(outs[i], i < 2 ? 2 : 1);
            for (size_t r = 0; r < got.size(); ++r) CHECK(std::memcmp(&got[r], &output[r], sizeof(float)) == 0);
            HIP_OK(hipFree(outs[i]));
        }
    }

    // batch_mv: three identical tokens give the matvec result per token.
    float batch_input[3 * 64];
    for (int t = 0; t < 3; ++t) std::memcpy(batch_input + 64 * t, input, sizeof(input));
    auto* device_batch = device_copy(batch_input, 3 * 64);
    float* device_batch_out = device_floats(3 * 2);
    qwen3x_hip::batch_mv(matrix, device_batch, device_batch_out, 3, false, nullptr);
    const auto batch = host_copy(device_batch_out, 6);
    for (int t = 0; t < 3; ++t)
        for (int row = 0; row < 2; ++row) CHECK(std::abs(batch[2 * t + row] - expected[row]) < 1e-6f);
    HIP_OK(hipFree(weight)); HIP_OK(hipFree(device_input)); HIP_OK(hipFree(device_output));
    HIP_OK(hipFree(device_embedding)); HIP_OK(hipFree(device_batch)); HIP_OK(hipFree(device_batch_out));
}

// tests/q4_cpu_test.cpp:138-178
void q4_math_test() {
    Q4Block blocks[4]{};
    const uint16_t scales[4] = {0x3c00, 0x3800, 0x4000, 0x3400};
    for (int block = 0; block < 4; ++block) {
        blocks[block].scale = scales[block];
        for (int index = 0; index < 16; ++index) {
            const int low = (index + block) % 16;
            const int high = (15 - index + block) % 16;
            blocks[block].values[index] = static_cast<uint8_t>(low | (high << 4));
        }
    }
    float input[64];
    for (int index = 0; index < 64; ++index) input[index] = (index % 7 - 3) * 0.125f;
    const float decoded_scales[4] = {1.0f, 0.5f, 2.0f, 0.25f};
    float expected[2]{};
    for (int row = 0; row < 2; ++row)
        for (int block = 0; block < 2; ++block)
            for (int index = 0; index < 16; ++index) {
                const uint8_t packed = blocks[row * 2 + block].values[index];
                expected[row] += decoded_scales[row * 2 + block] * ((packed & 15) - 8) * input[block * 32 + index];
                expected[row] += decoded_scales[row * 2 + block] * ((packed >> 4) - 8) * input[block * 32 + index + 16];
            }
    auto* weight = device_copy(blocks, 4);
    auto* device_input = device_copy(input, 64);
    float* device_output = device_floats(2);
    const qwen3x_hip::Linear matrix{weight, 2, 64, qwen3x_hip::MATRIX_Q4_0};
    qwen3x_hip::mv(matrix, device_input, device_output, nullptr);
    const auto output = host_copy(device_output, 2);
    CHECK(std::abs(output[0] - expected[0]) < 1e-6f);
    CHECK(std::abs(output[1] - expected[1]) < 1e-6f);
    float* device_embedding = device_floats(64);
    qwen3x_hip::embed(matrix, 1, device_embedding, nullptr);
    const auto embedding = host_copy(device_embedding, 64);
    for (int index = 0; index < 16; ++index) {
        const uint8_t low = blocks[2].values[index] & 15;
        const uint8_t high = blocks[2].values[index] >> 4;
        CHECK(embedding[index] == 2.0f * (low - 8));
        CHECK(embedding[index + 16] == 2.0f * (high - 8));
    }
    HIP_OK(hipFree(weight)); HIP_OK(hipFree(device_input)); HIP_OK(hipFree(device_output));
    HIP_OK(hipFree(device_embedding));
}

// tests/q4_cuda_test.cu:109-131 (and q4_cpu_test.cpp:180-202 for the six-logit case)
void router_test() {
    float logits[256];
    for (int expert = 0; expert < 256; ++expert) logits[expert] = expert * 0.03125f;
    auto* device_logits = device_copy(logits, 256);
    int* ids = nullptr;
    float* weights = device_floats(8);
    HIP_OK(hipMalloc(&ids, 8 * sizeof(int)));
    qwen3x_hip::router_top_k(device_logits, 1, 256, 8, ids, weights, nullptr);
    const auto host_ids = host_copy(ids, 8);
    const auto host_weights = host_copy(weights, 8);
    float sum = 0.0f;
    for (int slot = 0; slot < 8; ++slot) {
        CHECK(host_ids[slot] == 255 - slot);
        sum += host_weights[slot];
    }
    CHECK(std::abs(sum - 1.0f) < 1e-6f);

    const float six[6] = {-2.0f, 3.0f, 1.0f, 4.0f, -1.0f, 2.0f};
    auto* device_six = device_copy(six, 6);
    qwen3x_hip::router_top_k(device_six, 1, 6, 3, ids, weights, nullptr);
    const auto six_ids = host_copy(ids, 3);
    const auto six_weights = host_copy(weights, 3);
    CHECK(six_ids[0] == 3 && six_ids[1] == 1 && six_ids[2] == 5);
    CHECK(std::abs(six_weights[0] + six_weights[1] + six_weights[2] - 1.0f) < 1e-6f);
    HIP_OK(hipFree(device_logits)); HIP_OK(hipFree(device_six)); HIP_OK(hipFree(ids)); HIP_OK(hipFree(weights));
}

// tests/q4_cuda_test.cu:62-107: constant 0x99 nibbles (value 1) give closed
// forms.  Run once as decode (1 token) and once grouped (3 equal tokens).
void expert_moe_test() {
    constexpr int EXPERTS = 4, TOP_K = 2, H = 32, I = 32;
    const uint16_t scales[EXPERTS] = {0x3400, 0x3800, 0x3c00, 0x4000};
    std::vector<Q4Block> host_gate(EXPERTS * 2 * I), host_down(EXPERTS * H);
    for (int expert = 0; expert < EXPERTS; ++expert) {
        for (int row = 0; row < 2 * I; ++row) {
            host_gate[expert * 2 * I + row].scale = scales[expert];
            std::memset(host_gate[expert * 2 * I + row].values, 0x99, 16);
        }
        for (int row = 0; row < H; ++row) {
            host_down[expert * H + row].scale = scales[expert];
            std::memset(host_down[expert * H + row].values, 0x99, 16);
        }
    }
    auto* gate = device_copy(host_gate.data(), host_gate.size());
    auto* down = device_copy(host_down.data(), host_down.size());
    const float input_sum = 16.5f;
    const float gate2 = input_sum, gate1 = input_sum * 0.5f;
    const float hidden2 = silu(gate2) * gate2, hidden1 = silu(gate1) * gate1;
    const float routing[TOP_K] = {0.75f, 0.25f};
    const float expected = routing[0] * I * hidden2 + routing[1] * 0.5f * I * hidden1;
    const qwen3x_hip::ExpertLinear gu{gate, EXPERTS, 2 * I, H, qwen3x_hip::MATRIX_Q4_0};
    const qwen3x_hip::ExpertLinear dn{down, EXPERTS, H, I, qwen3x_hip::MATRIX_Q4_0};
    for (int tokens : {1, 3}) {
        std::vector<float> input(tokens * H);
        std::vector<int> ids(tokens * TOP_K);
        std::vector<float> weights(tokens * TOP_K);
        for (int t = 0; t < tokens; ++t) {
            for (int i = 0; i < H; ++i) input[t * H + i] = 0.03125f * (i + 1);
            ids[t * TOP_K] = 2; ids[t * TOP_K + 1] = 1;
            weights[t * TOP_K] = routing[0]; weights[t * TOP_K + 1] = routing[1];
        }
        auto* device_input = device_copy(input.data(), input.size());
        auto* device_ids = device_copy(ids.data(), ids.size());
        auto* device_weights = device_copy(weights.data(), weights.size());
        float* output = device_floats(tokens * H);
        const size_t ws_bytes = qwen3x_hip::moe_workspace_bytes(tokens, EXPERTS, TOP_K, H, I);
        void* ws = nullptr;
        HIP_OK(hipMalloc(&ws, ws_bytes));
        qwen3x_hip::moe_routed(gu, dn, device_input, tokens, device_ids, device_weights, TOP_K, output, false,
                               ws, ws_bytes, nullptr);
        const auto actual = host_copy(output, tokens * H);
        for (float v : actual) {
            CHECK(std::isfinite(v));
            CHECK(std::abs(v - expected) < 1e-2f);
        }
        HIP_OK(hipFree(device_input)); HIP_OK(hipFree(device_ids)); HIP_OK(hipFree(device_weights));
        HIP_OK(hipFree(output)); HIP_OK(hipFree(ws));
    }
    HIP_OK(hipFree(gate)); HIP_OK(hipFree(down));
}

uint16_t bf16(float value) {  // tests/q4_cpu_test.cpp:203-208
    uint32_t bits = 0;
    std::memcpy(&bits, &value, sizeof(bits));
    return static_cast<uint16_t>(bits >> 16);
}

float sigmoid(float x) {  // engine.cpp:187-190
    if (x >= 0.0f) return 1.0f / (1.0f + std::exp(-x));
    const float e = std::exp(x);
    return e / (1.0f + e);
}

void fill_constant_q4(Q4Block* blocks, size_t count, uint16_t scale) {
    for (size_t i = 0; i < count; ++i) {
        blocks[i].scale = scale;
        std::memset(blocks[i].values, 0x99, sizeof(blocks[i].values));
    }
}

// tests/q4_cpu_test.cpp:217-276 (moe_test): the whole layer -- BF16 router,
// constant 0x99 experts, shared expert and its sigmoid gate -- against the
// closed form, through qwen3x_hip::moe (one token, then three equal tokens).
void moe_layer_test() {
    constexpr int EXPERTS = 4, TOP_K = 2, H = 32, I = 32;
    std::vector<uint16_t> router(EXPERTS * H);
    const float router_values[EXPERTS] = {-0.125f, 0.0625f, 0.125f, -0.0625f};
    for (int e = 0; e < EXPERTS; ++e)
        for (int c = 0; c < H; ++c) router[e * H + c] = bf16(router_values[e]);
    std::vector<Q4Block> gate_up(EXPERTS * 2 * I), down(EXPERTS * H);
    const uint16_t scales[EXPERTS] = {0x3400, 0x3800, 0x3c00, 0x4000};
    for (int e = 0; e < EXPERTS; ++e) {
        fill_constant_q4(gate_up.data() + e * 2 * I, 2 * I, scales[e]);
        fill_constant_q4(down.data() + e * H, H, scales[e]);
    }
    std::vector<Q4Block> shared_gate(I), shared_up(I), shared_down(H);
    fill_constant_q4(shared_gate.data(), I, 0x3400);
    fill_constant_q4(shared_up.data(), I, 0x3400);
    fill_constant_q4(shared_down.data(), H, 0x3400);
    std::vector<uint16_t> shared_scale(H, bf16(0.03125f));

    const qwen3x_hip::MatrixType q4 = qwen3x_hip::MATRIX_Q4_0, b16 = qwen3x_hip::MATRIX_BF16;
    auto* d_router = device_copy(router.data(), router.size());
    auto* d_gate_up = device_copy(gate_up.data(), gate_up.size());
    auto* d_down = device_copy(down.data(), down.size());
    auto* d_sg = device_copy(shared_gate.data(), shared_gate.size());
    auto* d_su = device_copy(shared_up.data(), shared_up.size());
    auto* d_sd = device_copy(shared_down.data(), shared_down.size());
    auto* d_scale = device_copy(shared_scale.data(), shared_scale.size());
    const qwen3x_hip::MoeWeights weights{
        {d_router, EXPERTS, H, b16}, {d_gate_up, EXPERTS, 2 * I, H, q4}, {d_down, EXPERTS, H, I, q4},
        {d_sg, I, H, q4},            {d_su, I, H, q4},                    {d_sd, H, I, q4},
        {d_scale, 1, H, b16},
    };

    const float logits[EXPERTS] = {-4.0f, 2.0f, 4.0f, -2.0f};
    const float p1 = std::exp(logits[1] - logits[2]);
    const float expert1 = 0.5f * I * silu(0.5f * H) * (0.5f * H);
    const float expert2 = 1.0f * I * silu(1.0f * H) * (1.0f * H);
    const float routed = (p1 * expert1 + expert2) / (p1 + 1.0f);
    const float shared_hidden = silu(0.25f * H) * (0.25f * H);
    const float shared = sigmoid(1.0f) * 0.25f * I * shared_hidden;
    const float expected = routed + shared;
    for (int tokens : {1, 3}) {
        std::vector<float> input(tokens * H, 1.0f);
        auto* d_input = device_copy(input.data(), input.size());
        float* output = device_floats(tokens * H);
        int* ids = nullptr;
        HIP_OK(hipMalloc(&ids, tokens * TOP_K * sizeof(int)));
        const size_t ws_bytes = qwen3x_hip::moe_workspace_bytes(weights, TOP_K, tokens);
        void* ws = nullptr;
        HIP_OK(hipMalloc(&ws, ws_bytes));
        qwen3x_hip::moe(weights, d_input, tokens, output, TOP_K, ids, nullptr, ws, ws_bytes, nullptr);
        const auto actual = host_copy(output, tokens * H);
        const auto chosen = host_copy(ids, tokens * TOP_K);
        for (int t = 0; t < tokens; ++t) CHECK(chosen[t * TOP_K] == 2 && chosen[t * TOP_K + 1] == 1);
        for (float v : actual) {
            CHECK(std::isfinite(v));
            CHECK(std::abs(v - expected) < 1e-2f);
        }
        HIP_OK(hipFree(d_input)); HIP_OK(hipFree(output)); HIP_OK(hipFree(ids)); HIP_OK(hipFree(ws));
    }
    for (void* p : {static_cast<void*>(d_router), static_cast<void*>(d_gate_up), static_cast<void*>(d_down),
                    static_cast<void*>(d_sg), static_cast<void*>(d_su), static_cast<void*>(d_sd),
                    static_cast<void*>(d_scale)})
        HIP_OK(hipFree(p));
}

// ---- model.bin loader (q8_cpu_test.cpp:222-264, q4_cpu_test.cpp:85-136) ----

// The 72-byte header of a model: magic, then the 16 fields (model_config.h:
// 22-39, values :77-93).
std::vector<uint8_t> model_header(const uint32_t (&fields)[16]) {
    std::vector<uint8_t> header(72, 0);
    std::memcpy(header.data(), "Q3XMODL\0", 8);
    std::memcpy(header.data() + 8, fields, sizeof(fields));
    return header;
}

void pwrite_exact(int fd, const void* data, size_t size, off_t offset) {
    CHECK(pwrite(fd, data, size, offset) == static_cast<ssize_t>(size));
}

void check_loader(const char* path, bool expected, const char* expected_error) {
    qwen3x_hip::Model model;
    const char* error = nullptr;
    CHECK(model.load(path, &error) == expected);
    if (expected) {
        CHECK(error == nullptr);
    } else {
        CHECK(error != nullptr && std::strstr(error, expected_error) != nullptr);
        CHECK(model.handle == nullptr && model.layers == nullptr);
    }
}

void loader_test_q8_9b() {
    const uint32_t fields[16] = {9000, 248320, 4096, 12288, 32, 4, 16, 4, 256, 64, 16, 32, 128, 128, 4, 262144};
    const auto header = model_header(fields);
    const size_t expected_size = 9514418816ULL;  // q8_cpu_test.cpp:228
    char path[] = "/tmp/q3x-hip-q8-loader-XXXXXX";
    const int fd = mkstemp(path);
    CHECK(fd >= 0);
    auto restore = [&]() {
        CHECK(ftruncate(fd, static_cast<off_t>(expected_size)) == 0);
        pwrite_exact(fd, header.data(), header.size(), 0);
    };
    restore();
    {
        qwen3x_hip::Model model;
        const char* error = nullptr;
        CHECK(model.load(path, &error));
        CHECK(model.config.id == 9000 && model.config.matrix_type == Q3X_HIP_MATRIX_Q8_0);
        CHECK(model.lm_head.weight != model.embedding.weight && model.lm_head.rows == 248320);
        CHECK(model.layers[0].gate.rows == 12288 && model.layers[0].gate.columns == 4096);
        CHECK(model.layers[31].down.rows == 4096 && model.layers[31].down.columns == 12288);
        CHECK(model.layers[3].attention.q.rows == 2 * 16 * 256 && model.layers[3].attention.qnorm);
        CHECK(model.layers[2].delta.qkv.rows == 2 * 16 * 128 + 32 * 128 && model.layers[2].delta.alog);
        // Every weight is 64-byte aligned inside the one device buffer.
        CHECK(reinterpret_cast<uintptr_t>(model.layers[7].delta.norm) % 64 == 0);
    }
    CHECK(ftruncate(fd, static_cast<off_t>(expected_size - 1)) == 0);
    check_loader(path, false, "truncated");
    restore();
    CHECK(ftruncate(fd, static_cast<off_t>(expected_size + 1)) == 0);
    check_loader(path, false, "size does not match schema");
    restore();
    const uint8_t wrong_magic = 'X';
    pwrite_exact(fd, &wrong_magic, 1, 0);
    check_loader(path, false, "wrong model.bin magic");
    restore();
    const uint32_t unknown_id = 9001;
    pwrite_exact(fd, &unknown_id, 4, 8);
    check_loader(path, false, "unsupported Qwen model ID");
    restore();
    const uint32_t wrong_hidden = 4095;
    pwrite_exact(fd, &wrong_hidden, 4, 8 + 2 * 4);
    check_loader(path, false, "header mismatch");
    close(fd);
    CHECK(unlink(path) == 0);
}

void loader_test_q4_35b() {
    const uint32_t fields[16] = {36035, 248320, 2048, 512, 40, 4, 16, 2, 256, 64, 16, 32, 128, 128, 4, 262144};
    const auto header = model_header(fields);
    const size_t expected_size = 19528534784ULL;  // q4_cpu_test.cpp:15
    char path[] = "/tmp/q3x-hip-q4-loader-XXXXXX";
    const int fd = mkstemp(path);
    CHECK(fd >= 0);
    auto restore = [&]() {
        CHECK(ftruncate(fd, static_cast<off_t>(expected_size)) == 0);
        pwrite_exact(fd, header.data(), header.size(), 0);
    };
    restore();
    {
        qwen3x_hip::Model model;
        const char* error = nullptr;
        CHECK(model.load(path, &error));
        CHECK(error == nullptr);
        CHECK(model.config.id == 36035);
        CHECK(model.layers[39].moe.gate_up.experts == 256);
        CHECK(model.layers[39].moe.gate_up.rows == 1024 && model.layers[39].moe.down.columns == 512);
        CHECK(model.layers[0].moe.router.type == qwen3x_hip::MATRIX_BF16 && model.layers[0].moe.router.rows == 256);
        CHECK(model.layers[0].moe.shared_scale.rows == 1 && model.layers[0].moe.shared_down.columns == 512);
    }
    auto reject_header = [&](off_t offset, uint32_t value, const char* expected) {
        restore();
        pwrite_exact(fd, &value, sizeof(value), offset);
        check_loader(path, false, expected);
    };
    reject_header(0, 0, "magic");
    reject_header(8, 12345, "model ID");
    reject_header(8 + 4, 1, "header mismatch");
    restore();
    CHECK(ftruncate(fd, static_cast<off_t>(expected_size - 1)) == 0);
    check_loader(path, false, "truncated");
    restore();
    CHECK(ftruncate(fd, static_cast<off_t>(expected_size + 1)) == 0);
    check_loader(path, false, "size does not match schema");
    check_loader("/nonexistent/model.bin", false, "cannot open model.bin");
    close(fd);
    CHECK(unlink(path) == 0);
}

// The backend operations (internal.h:11-34) on a sparse full-size 9B file:
// all-zero weights give all-zero logits, so argmax is 0; the life cycle,
// checkpoints and constants follow the reference's backends.
void backend_test() {
    const uint32_t fields[16] = {9000, 248320, 4096, 12288, 32, 4, 16, 4, 256, 64, 16, 32, 128, 128, 4, 262144};
    const auto header = model_header(fields);
    char path[] = "/tmp/q3x-hip-backend-XXXXXX";
    const int fd = mkstemp(path);
    CHECK(fd >= 0);
    CHECK(ftruncate(fd, static_cast<off_t>(9514418816ULL)) == 0);
    pwrite_exact(fd, header.data(), header.size(), 0);
    char err[128] = "x";
    CHECK(q3x_backend::model_create("/nonexistent/model.bin", err, sizeof(err)) == nullptr);
    CHECK(std::strstr(err, "cannot open model.bin") != nullptr);
    q3x_backend::Model* model = q3x_backend::model_create(path, err, sizeof(err));
    CHECK(model != nullptr && err[0] == '\0');
    CHECK(q3x_backend::model_id(model) == 9000);
    q3x_backend::State* state = q3x_backend::state_create(model, 16);
    const int tokens[3] = {1, 248043, 7};
    q3x_backend::state_forward(model, state, tokens, 3, true);
    std::vector<float> logits(248320, 1.0f);
    q3x_backend::state_copy_logits(state, logits.data());
    for (float v : logits) CHECK(v == 0.0f);
    CHECK(q3x_backend::state_argmax(state) == 0);
    q3x_backend::state_checkpoint_save(state);
    q3x_backend::state_forward(model, state, tokens, 1, true);
    q3x_backend::state_checkpoint_restore(state);
    q3x_backend::state_reset(state);
    q3x_backend::state_forward(model, state, tokens + 2, 1, false);
    CHECK(q3x_backend::vocab_size() == 248320 && q3x_backend::max_context() == 262144);
    CHECK(q3x_backend::token_is_stop(248044) && q3x_backend::token_is_stop(248046) &&
          !q3x_backend::token_is_stop(248045));
    q3x_backend::state_destroy(state);
    q3x_backend::model_destroy(model);
    close(fd);
    CHECK(unlink(path) == 0);
}

}  // namespace

int main() {
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
        std::puts("q3x-hip-host-test: skipped (no GPU)");
        return 77;
    }
    q4_mv_test();
    q8_fixed_test();
    q4_math_test();
    router_test();
    expert_moe_test();
    moe_layer_test();
    loader_test_q8_9b();
    loader_test_q4_35b();
    backend_test();
    HIP_OK(hipDeviceSynchronize());
    std::puts("q3x-hip-host-test: ok");
    return 0;
}
