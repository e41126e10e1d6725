// engine.hip -- the decode engine: tokens through every layer of a Q8_0 /
// Q4_0 Qwen3.5 / 3.6 / 3.8 model on the GPU, the caller of the matmul path.
//
// Follows the reference's forward (engine.cpp:431-454) layer for layer:
// embedding; per layer RMSNorm, the mixer (gated DeltaNet, engine.cpp:
// 274-316, or full attention, :318-362), residual, RMSNorm, FFN or MoE,
// residual; final RMSNorm and lm_head.  The matrices go through this
// library's own entry points (q3x_hip_mv_multi for the projection groups,
// q3x_hip_mv with accumulate for the output projections, which adds the
// residual in the same operation, q3x_hip_moe_layer for MoE layers); the
// kernels here are the small per-token operations between them.
//
// Every buffer lives on the device for the life of the engine: the work
// vectors, the DeltaNet recurrent state (conv history and the KD x VD memory
// of each head), the KV cache, the logits.  The token and the position are
// read from device memory, so one decode step is position-independent and
// is captured once into a hipGraph (two: with and without logits) and
// replayed for every token, as the reference captures its step
// (arch/cuda/engine.cu:1995-2005).
#include <math.h>

#include <algorithm>
#include <new>
#include <vector>

#include "common.h"
#include "rows.h"

struct q3x_hip_engine;

namespace q3x {
namespace {

constexpr float kEps = 1e-6f;           // engine.cpp:26 EPS
constexpr float kTheta = 10000000.0f;   // engine.cpp:26 THETA
constexpr int kNormThreads = 1024;
constexpr int kHeadThreads = 256;

__device__ __forceinline__ float bf16_value(uint16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }

// Sum over the workgroup in a fixed order: each wave's DPP sum, then the
// wave partials in wave order.  Every thread receives the total.
template <int THREADS>
__device__ float block_sum(float v, float* partial) {
    const float w = wave_sum_f32(v);
    if ((threadIdx.x & (kWave - 1)) == 0) partial[threadIdx.x / kWave] = w;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < THREADS / kWave; ++i) total += partial[i];
    __syncthreads();
    return total;
}
template <int THREADS>
__device__ float block_max(float v, float* partial) {
    const float w = wave_max_f32(v);
    if ((threadIdx.x & (kWave - 1)) == 0) partial[threadIdx.x / kWave] = w;
    __syncthreads();
    float m = partial[0];
#pragma unroll
    for (int i = 1; i < THREADS / kWave; ++i) m = fmaxf(m, partial[i]);
    __syncthreads();
    return m;
}

// engine.cpp:192
__device__ __forceinline__ float softplus_ref(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// Row `*token` of the embedding, dequantised bit for bit as the reference's
// embed (engine.cpp:195-200 via arch/cpu.cpp:55-63, 81-90).
template <uint32_t QT>
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t* __restrict__ w, int cols,
                                                    const int* __restrict__ tokens, const int* __restrict__ step,
                                                    float* __restrict__ out) {
    constexpr int BB = QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : kQ4Bytes;
    const int token = tokens[*step];
    const int bpr = cols / kBlock;
    const uint8_t* row = w + static_cast<size_t>(token) * bpr * BB;
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += gridDim.x * blockDim.x) {
        const uint8_t* blk = row + (c / kBlock) * BB;
        const float scale = f16_exact(blk[0] | (blk[1] << 8));
        const int within = c % kBlock;
        int q;
        if (QT == Q3X_HIP_MATRIX_Q8_0) {
            q = static_cast<int8_t>(blk[2 + within]);
        } else {
            const uint32_t packed = blk[2 + within % 16];
            q = static_cast<int>(within < 16 ? (packed & 15u) : (packed >> 4)) - 8;
        }
        out[c] = scale * static_cast<float>(q);
    }
}

// out = RMSNorm(hidden) * (1 + w) (engine.cpp:228-233); with `branch`,
// hidden += branch first and is written back (the residual add of
// engine.cpp:240-242 that precedes the norm).  One workgroup.
__global__ __launch_bounds__(kNormThreads) void rms_kernel(float* __restrict__ hidden, const float* __restrict__ branch,
                                                           const uint16_t* __restrict__ w, int n,
                                                           float* __restrict__ out) {
    __shared__ float partial[kNormThreads / kWave];
    float square = 0.0f;
    for (int i = threadIdx.x; i < n; i += kNormThreads) {
        float x = hidden[i];
        if (branch) {
            x += branch[i];
            hidden[i] = x;
        }
        square = fmaf(x, x, square);
    }
    const float total = block_sum<kNormThreads>(square, partial);
    const float scale = 1.0f / sqrtf(total / static_cast<float>(n) + kEps);
    for (int i = threadIdx.x; i < n; i += kNormThreads) out[i] = hidden[i] * scale * (1.0f + bf16_value(w[i]));
}

// Causal depthwise convolution of one token over the DQKV channels with
// CK - 1 remembered inputs, then SiLU (engine.cpp:251-261).
__global__ __launch_bounds__(256) void delta_conv_kernel(float* __restrict__ qkv, const uint16_t* __restrict__ w,
                                                         float* __restrict__ history, int channels, int CK) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= channels) return;
    const float x = qkv[c];
    const uint16_t* wc = w + static_cast<size_t>(c) * CK;
    float* past = history + static_cast<size_t>(c) * (CK - 1);
    float sum = x * bf16_value(wc[CK - 1]);
    for (int i = 0; i < CK - 1; ++i) sum = fmaf(past[i], bf16_value(wc[i]), sum);
    for (int i = 0; i < CK - 2; ++i) past[i] = past[i + 1];
    past[CK - 2] = x;
    qkv[c] = silu_ref(sum);
}

// One value head of the gated delta rule (engine.cpp:262-316): L2-normalised
// q and k of its key head (q also divided by sqrt(KD)), beta = sigmoid(b),
// decay = -exp(A_log) * softplus(a + dt_bias); the KD x VD memory S decays
// by exp(decay), takes k (beta (v - k S)), and gives out = q S; then the
// gated RMSNorm with the FP32 norm weight and SiLU(z) (engine.cpp:234-239).
// 256 threads: thread t owns value column t % 128 and half of the keys, so
// its S entries stay in registers between the three passes.
// Requires KD <= 128, VD <= 128.
__global__ __launch_bounds__(kHeadThreads) void delta_rule_kernel(
    const float* __restrict__ qkv, const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ z, const float* __restrict__ alog, const uint16_t* __restrict__ dt,
    const float* __restrict__ norm, float* __restrict__ memory, float* __restrict__ out, int KH, int VH, int KD,
    int VD) {
    __shared__ float qs[128], ks[128], part[2][128], partial[kHeadThreads / kWave];
    const int head = blockIdx.x;
    const int t = threadIdx.x;
    const int DQK = KH * KD;
    const int kh = head / (VH / KH);
    const float qv = t < KD ? qkv[kh * KD + t] : 0.0f;
    const float kv = t < KD ? qkv[DQK + kh * KD + t] : 0.0f;
    const float qn = block_sum<kHeadThreads>(qv * qv, partial);
    const float kn = block_sum<kHeadThreads>(kv * kv, partial);
    if (t < KD) {
        qs[t] = qv * (1.0f / sqrtf(qn + kEps)) / sqrtf(static_cast<float>(KD));
        ks[t] = kv * (1.0f / sqrtf(kn + kEps));
    }
    __syncthreads();
    const float beta = sigmoid_ref(b[head]);
    const float decay = -expf(alog[head]) * softplus_ref(a[head] + bf16_value(dt[head]));
    const float scale = expf(decay);
    const int v = t & 127, half = t >> 7;
    const int k0 = half * 64;
    const bool col = v < VD;
    float* S = memory + static_cast<size_t>(head) * KD * VD;
    float s[64];
    float pred = 0.0f;
#pragma unroll
    for (int j = 0; j < 64; ++j) {
        const int key = k0 + j;
        s[j] = col && key < KD ? S[static_cast<size_t>(key) * VD + v] * scale : 0.0f;
        if (key < KD) pred = fmaf(ks[key], s[j], pred);
    }
    part[half][v] = pred;
    __syncthreads();
    const float vv = col ? qkv[2 * DQK + head * VD + v] : 0.0f;
    const float delta = vv - (part[0][v] + part[1][v]);
    float o = 0.0f;
#pragma unroll
    for (int j = 0; j < 64; ++j) {
        const int key = k0 + j;
        if (key < KD) {
            s[j] = fmaf(ks[key] * beta, delta, s[j]);
            o = fmaf(qs[key], s[j], o);
            if (col) S[static_cast<size_t>(key) * VD + v] = s[j];
        }
    }
    __syncthreads();
    part[half][v] = o;
    __syncthreads();
    const float result = col && half == 0 ? part[0][v] + part[1][v] : 0.0f;
    const float sq = block_sum<kHeadThreads>(result * result, partial);
    if (col && half == 0) {
        const float g = 1.0f / sqrtf(sq / static_cast<float>(VD) + kEps);
        out[head * VD + v] = result * (g * norm[v] * silu_ref(z[head * VD + v]));
    }
}

// RMSNorm (1 + w) and rotary embedding of one AD-wide head at `position`
// (engine.cpp:228-233, 243-250), in place in `x` (shared memory).
__device__ void norm_rope(float* x, const uint16_t* w, int AD, int RD, int position, float* partial) {
    const int t = threadIdx.x;
    const float v = t < AD ? x[t] : 0.0f;
    const float sq = block_sum<kHeadThreads>(v * v, partial);
    const float scale = 1.0f / sqrtf(sq / static_cast<float>(AD) + kEps);
    const float y = t < AD ? v * scale * (1.0f + bf16_value(w[t])) : 0.0f;
    if (t < AD) x[t] = y;
    __syncthreads();
    float r = y;
    const int h = RD / 2;
    if (t < RD) {
        const int i = t < h ? t : t - h;
        const float angle = static_cast<float>(position) / powf(kTheta, 2.0f * static_cast<float>(i) / static_cast<float>(RD));
        const float c = cosf(angle), s = sinf(angle);
        r = t < h ? x[t] * c - x[t + h] * s : x[t] * c + x[t - h] * s;
    }
    __syncthreads();
    if (t < RD) x[t] = r;
    __syncthreads();
}

// Query heads (blocks 0 .. AH-1): split the q|gate rows, norm and rotate q;
// key/value heads (blocks AH ..): norm and rotate k and append k and v to
// the cache at the current position (engine.cpp:318-343).  AD <= 256.
__global__ __launch_bounds__(kHeadThreads) void attention_prep_kernel(
    const float* __restrict__ query_and_gate, const float* __restrict__ key, const float* __restrict__ value,
    const uint16_t* __restrict__ qnorm, const uint16_t* __restrict__ knorm, const int* __restrict__ position,
    float* __restrict__ query, float* __restrict__ gate, float* __restrict__ key_cache,
    float* __restrict__ value_cache, int AH, int KVH, int AD, int RD) {
    __shared__ float x[256], partial[kHeadThreads / kWave];
    const int t = threadIdx.x;
    const int pos = *position;
    if (blockIdx.x < AH) {
        const int head = blockIdx.x;
        if (t < AD) {
            x[t] = query_and_gate[head * 2 * AD + t];
            gate[head * AD + t] = query_and_gate[head * 2 * AD + AD + t];
        }
        __syncthreads();
        norm_rope(x, qnorm, AD, RD, pos, partial);
        if (t < AD) query[head * AD + t] = x[t];
    } else {
        const int head = blockIdx.x - AH;
        if (t < AD) x[t] = key[head * AD + t];
        __syncthreads();
        norm_rope(x, knorm, AD, RD, pos, partial);
        const size_t at = (static_cast<size_t>(pos) * KVH + head) * AD;
        if (t < AD) {
            key_cache[at + t] = x[t];
            value_cache[at + t] = value[head * AD + t];
        }
    }
}

// One query head over positions 0 .. position (engine.cpp:344-361): scores
// q . k / sqrt(AD), max-subtracted softmax, sum of p / total * v in token
// order, times sigmoid(gate).  Scores go to `scores` [AH, capacity].
__global__ __launch_bounds__(kHeadThreads) void attention_kernel(
    const float* __restrict__ query, const float* __restrict__ gate, const float* __restrict__ key_cache,
    const float* __restrict__ value_cache, const int* __restrict__ position, float* __restrict__ scores,
    float* __restrict__ out, int AH, int KVH, int AD, int capacity) {
    __shared__ float partial[kHeadThreads / kWave];
    const int head = blockIdx.x;
    const int kv = head / (AH / KVH);
    const int n = *position + 1;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const float* q = query + head * AD;
    float* sc = scores + static_cast<size_t>(head) * capacity;
    const float divisor = sqrtf(static_cast<float>(AD));
    float qr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) qr[j] = lane + 64 * j < AD ? q[lane + 64 * j] : 0.0f;
    for (int tok = wave; tok < n; tok += kHeadThreads / kWave) {
        const float* k = key_cache + (static_cast<size_t>(tok) * KVH + kv) * AD;
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + 64 * j < AD) d = fmaf(qr[j], k[lane + 64 * j], d);
        d = wave_sum_f32(d);
        if (lane == 0) sc[tok] = d / divisor;
    }
    __syncthreads();
    float m = -INFINITY;
    for (int tok = threadIdx.x; tok < n; tok += kHeadThreads) m = fmaxf(m, sc[tok]);
    m = block_max<kHeadThreads>(m, partial);
    float sum = 0.0f;
    for (int tok = threadIdx.x; tok < n; tok += kHeadThreads) {
        const float e = expf(sc[tok] - m);
        sc[tok] = e;
        sum += e;
    }
    const float total = block_sum<kHeadThreads>(sum, partial);  // also orders the sc writes before the reads
    const int i = threadIdx.x;
    if (i < AD) {
        float acc = 0.0f;
        for (int tok = 0; tok < n; ++tok)
            acc = fmaf(sc[tok] / total, value_cache[(static_cast<size_t>(tok) * KVH + kv) * AD + i], acc);
        out[head * AD + i] = acc * sigmoid_ref(gate[head * AD + i]);
    }
}

// h = silu(gate) * up (engine.cpp:371-376), in place in gate.
__global__ __launch_bounds__(256) void swiglu_kernel(float* __restrict__ gate, const float* __restrict__ up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) gate[i] = silu_ref(gate[i]) * up[i];
}

// The first index of the largest logit (std::max_element, engine.cpp:606-610).
__global__ __launch_bounds__(kNormThreads) void argmax_kernel(const float* __restrict__ x, int n, int* __restrict__ out) {
    __shared__ float bv[kNormThreads / kWave];
    __shared__ int bi[kNormThreads / kWave];
    float best = -INFINITY;
    int index = n;
    for (int i = threadIdx.x; i < n; i += kNormThreads)
        if (x[i] > best || index == n) { best = x[i]; index = i; }
    // Wave: the largest value, the lowest index among equals.
    for (int off = 32; off >= 1; off >>= 1) {
        const float ob = __shfl_xor(best, off);
        const int oi = __shfl_xor(index, off);
        if (ob > best || (ob == best && oi < index)) { best = ob; index = oi; }
    }
    if ((threadIdx.x & (kWave - 1)) == 0) {
        bv[threadIdx.x / kWave] = best;
        bi[threadIdx.x / kWave] = index;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = bv[0];
        int k = bi[0];
        for (int w = 1; w < kNormThreads / kWave; ++w)
            if (bv[w] > b || (bv[w] == b && bi[w] < k)) { b = bv[w]; k = bi[w]; }
        *out = k;
    }
}

// Moves to the next token: step (index into the token list) and position.
__global__ void advance_kernel(int* step, int* position) {
    *step += 1;
    *position += 1;
}
__global__ void set_counters_kernel(int* step, int* position, int step_value, int position_value) {
    *step = step_value;
    *position = position_value;
}

}  // namespace
}  // namespace q3x

using namespace q3x;

namespace {

struct Mat {
    const void* w = nullptr;
    int rows = 0, cols = 0;
};

struct LayerWeights {
    bool attention = false;
    const uint16_t *input_norm = nullptr, *post_norm = nullptr;
    Mat qkv, z, a, b, out;  // DeltaNet
    const uint16_t* conv = nullptr;
    const float* alog = nullptr;
    const uint16_t* dt = nullptr;
    const float* norm = nullptr;
    Mat q, k, v, o;  // attention
    const uint16_t *qnorm = nullptr, *knorm = nullptr;
    Mat gate, up, down;  // dense FFN
    q3x_hip_moe_layer_weights moe{};
    float* conv_state = nullptr;  // DeltaNet: [DQKV, CK - 1]
    float* memory = nullptr;      //           [VH, KD, VD]
    float* key_cache = nullptr;   // attention: [capacity, KVH, AD]
    float* value_cache = nullptr;
};

bool engine_config_ok(const q3x_hip_model_config& c, int context) {
    return (c.matrix_type == Q3X_HIP_MATRIX_Q8_0 || c.matrix_type == Q3X_HIP_MATRIX_Q4_0) && c.KD <= 128 &&
           c.VD <= 128 && c.AD <= 256 && c.RD <= 64 && c.RD % 2 == 0 && c.RD <= c.AD && c.CK >= 2 && c.CK <= 8 &&
           c.top_k <= 8 && context >= 1 && context <= 262144;
}

}  // namespace

struct q3x_hip_engine {
    q3x_hip_model_config c{};
    int capacity = 0;
    int position = 0;             // host mirror of *d_position
    int checkpoint_position = 0;
    Mat embedding, lm_head;
    const uint16_t* final_norm = nullptr;
    std::vector<LayerWeights> layers;
    // device memory: one arena
    void* arena = nullptr;
    float *hidden = nullptr, *normalized = nullptr, *branch = nullptr, *logits = nullptr;
    float *qkv = nullptr, *z = nullptr, *a = nullptr, *b = nullptr, *delta_out = nullptr;
    float *query_and_gate = nullptr, *query = nullptr, *gate = nullptr, *key = nullptr, *value = nullptr;
    float *attn_out = nullptr, *scores = nullptr, *ffn_gate = nullptr, *ffn_up = nullptr;
    float *recurrent = nullptr, *checkpoint_recurrent = nullptr, *checkpoint_logits = nullptr;
    size_t recurrent_floats = 0;
    int *d_tokens = nullptr, *d_step = nullptr, *d_position = nullptr, *d_argmax = nullptr;
    void* moe_ws = nullptr;
    size_t moe_ws_bytes = 0;
    int* h_tokens = nullptr;  // pinned staging of a forward's tokens
    int token_capacity = 0;
    hipStream_t stream = nullptr;
    hipGraphExec_t graph[2] = {nullptr, nullptr};
};

namespace {

template <typename T>
T* carve(uint8_t*& cursor, size_t count) {
    T* p = reinterpret_cast<T*>(cursor);
    cursor += (count * sizeof(T) + 255) / 256 * 256;
    return p;
}

// Enqueues one decode step: token tokens[*d_step] at *d_position.
int enqueue_step(q3x_hip_engine& e, bool logits) {
    const q3x_hip_model_config& c = e.c;
    hipStream_t s = e.stream;
    const int DQKV = 2 * c.KH * c.KD + c.VH * c.VD;
    const uint32_t type = c.matrix_type;
    const int eb = (c.H + 255) / 256;
    if (type == Q3X_HIP_MATRIX_Q8_0)
        hipLaunchKernelGGL(embed_kernel<Q3X_HIP_MATRIX_Q8_0>, dim3(eb), dim3(256), 0, s,
                           static_cast<const uint8_t*>(e.embedding.w), c.H, e.d_tokens, e.d_step, e.hidden);
    else
        hipLaunchKernelGGL(embed_kernel<Q3X_HIP_MATRIX_Q4_0>, dim3(eb), dim3(256), 0, s,
                           static_cast<const uint8_t*>(e.embedding.w), c.H, e.d_tokens, e.d_step, e.hidden);
    int rc = launch_status();
    bool pending = false;  // an MoE output in `branch` still to be added to hidden
    for (int i = 0; i < c.N && rc == Q3X_HIP_OK; ++i) {
        const LayerWeights& L = e.layers[i];
        hipLaunchKernelGGL(rms_kernel, dim3(1), dim3(kNormThreads), 0, s, e.hidden, pending ? e.branch : nullptr,
                           L.input_norm, c.H, e.normalized);
        if (!L.attention) {
            const q3x_hip_mv_item items[4] = {{L.qkv.w, L.qkv.rows, e.qkv, 0},
                                              {L.z.w, L.z.rows, e.z, 0},
                                              {L.a.w, L.a.rows, e.a, 0},
                                              {L.b.w, L.b.rows, e.b, 0}};
            rc = q3x_hip_mv_multi(items, 4, type, c.H, e.normalized, s);
            if (rc) break;
            hipLaunchKernelGGL(delta_conv_kernel, dim3((DQKV + 255) / 256), dim3(256), 0, s, e.qkv, L.conv,
                               L.conv_state, DQKV, c.CK);
            hipLaunchKernelGGL(delta_rule_kernel, dim3(c.VH), dim3(kHeadThreads), 0, s, e.qkv, e.a, e.b, e.z,
                               L.alog, L.dt, L.norm, L.memory, e.delta_out, c.KH, c.VH, c.KD, c.VD);
            rc = q3x_hip_mv(L.out.w, type, L.out.rows, L.out.cols, e.delta_out, e.hidden, 1, s);
        } else {
            const q3x_hip_mv_item items[3] = {{L.q.w, L.q.rows, e.query_and_gate, 0},
                                              {L.k.w, L.k.rows, e.key, 0},
                                              {L.v.w, L.v.rows, e.value, 0}};
            rc = q3x_hip_mv_multi(items, 3, type, c.H, e.normalized, s);
            if (rc) break;
            hipLaunchKernelGGL(attention_prep_kernel, dim3(c.AH + c.KVH), dim3(kHeadThreads), 0, s,
                               e.query_and_gate, e.key, e.value, L.qnorm, L.knorm, e.d_position, e.query, e.gate,
                               L.key_cache, L.value_cache, c.AH, c.KVH, c.AD, c.RD);
            hipLaunchKernelGGL(attention_kernel, dim3(c.AH), dim3(kHeadThreads), 0, s, e.query, e.gate,
                               L.key_cache, L.value_cache, e.d_position, e.scores, e.attn_out, c.AH, c.KVH, c.AD,
                               e.capacity);
            rc = q3x_hip_mv(L.o.w, type, L.o.rows, L.o.cols, e.attn_out, e.hidden, 1, s);
        }
        if (rc) break;
        hipLaunchKernelGGL(rms_kernel, dim3(1), dim3(kNormThreads), 0, s, e.hidden, nullptr, L.post_norm, c.H,
                           e.normalized);
        if (c.experts) {
            rc = q3x_hip_moe_layer(&L.moe, e.normalized, 1, e.branch, nullptr, nullptr, e.moe_ws, e.moe_ws_bytes,
                                   s);
            pending = true;
        } else {
            const q3x_hip_mv_item items[2] = {{L.gate.w, L.gate.rows, e.ffn_gate, 0}, {L.up.w, L.up.rows, e.ffn_up, 0}};
            rc = q3x_hip_mv_multi(items, 2, type, c.H, e.normalized, s);
            if (rc) break;
            hipLaunchKernelGGL(swiglu_kernel, dim3((c.I + 255) / 256), dim3(256), 0, s, e.ffn_gate, e.ffn_up, c.I);
            rc = q3x_hip_mv(L.down.w, type, L.down.rows, L.down.cols, e.ffn_gate, e.hidden, 1, s);
            pending = false;
        }
        if (rc == Q3X_HIP_OK) rc = launch_status();
    }
    if (rc) return rc;
    if (logits) {
        hipLaunchKernelGGL(rms_kernel, dim3(1), dim3(kNormThreads), 0, s, e.hidden, pending ? e.branch : nullptr,
                           e.final_norm, c.H, e.normalized);
        rc = q3x_hip_mv(e.lm_head.w, type, e.lm_head.rows, e.lm_head.cols, e.normalized, e.logits, 0, s);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, e.d_step, e.d_position);
    return launch_status();
}

int capture(q3x_hip_engine& e, bool logits) {
    hipGraph_t g = nullptr;
    if (hipStreamBeginCapture(e.stream, hipStreamCaptureModeThreadLocal) != hipSuccess) return Q3X_HIP_ERUNTIME;
    const int rc = enqueue_step(e, logits);
    const hipError_t end = hipStreamEndCapture(e.stream, &g);
    if (rc != Q3X_HIP_OK || end != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return rc ? rc : Q3X_HIP_ERUNTIME;
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t inst = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (inst != hipSuccess) return Q3X_HIP_ERUNTIME;
    e.graph[logits ? 1 : 0] = exec;
    return Q3X_HIP_OK;
}

void set_error(const char** error, const char* message) {
    if (error) *error = message;
}

}  // namespace

extern "C" int q3x_hip_engine_reset(q3x_hip_engine* e);

extern "C" void q3x_hip_engine_destroy(q3x_hip_engine* e) {
    if (!e) return;
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    for (auto& g : e->graph)
        if (g) (void)hipGraphExecDestroy(g);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    if (e->h_tokens) (void)hipHostFree(e->h_tokens);
    if (e->arena) (void)hipFree(e->arena);
    delete e;
}

extern "C" int q3x_hip_engine_create(const q3x_hip_model_config* config, const void* weights, int context,
                                     q3x_hip_engine** engine, const char** error) {
    if (!config || !weights || !engine) return Q3X_HIP_EINVAL;
    *engine = nullptr;
    const q3x_hip_model_config& c = *config;
    size_t count = 0;
    if (q3x_hip_model_schema(config, nullptr, 0, &count, nullptr) != Q3X_HIP_OK) {
        set_error(error, "invalid model configuration");
        return Q3X_HIP_EINVAL;
    }
    if (!engine_config_ok(c, context)) {
        set_error(error, c.matrix_type == Q3X_HIP_MATRIX_BF16 ? "BF16 models are not handled by the HIP backend"
                                                              : "configuration outside the HIP engine's limits");
        return c.matrix_type == Q3X_HIP_MATRIX_BF16 ? Q3X_HIP_ENOTSUP : Q3X_HIP_EINVAL;
    }
    std::vector<q3x_hip_tensor> table(count);
    if (q3x_hip_model_schema(config, table.data(), count, &count, nullptr) != Q3X_HIP_OK) return Q3X_HIP_EINVAL;
    q3x_hip_engine* e = new (std::nothrow) q3x_hip_engine();
    if (!e) return Q3X_HIP_ERUNTIME;
    e->c = c;
    e->capacity = context;
    e->layers.resize(c.N);
    const uint8_t* base = static_cast<const uint8_t*>(weights);
    for (const auto& t : table) {
        const void* p = base + t.offset;
        const Mat m{p, t.rows * std::max(t.experts, 1), t.cols};
        const uint16_t* bf = static_cast<const uint16_t*>(p);
        const float* f32 = static_cast<const float*>(p);
        if (t.layer < 0) {
            if (t.role == Q3X_HIP_EMBEDDING) e->embedding = m;
            else if (t.role == Q3X_HIP_LM_HEAD) e->lm_head = m;
            else if (t.role == Q3X_HIP_FINAL_NORM) e->final_norm = bf;
            continue;
        }
        LayerWeights& L = e->layers[t.layer];
        switch (t.role) {
        case Q3X_HIP_INPUT_NORM: L.input_norm = bf; break;
        case Q3X_HIP_POST_NORM: L.post_norm = bf; break;
        case Q3X_HIP_DELTA_QKV: L.qkv = m; break;
        case Q3X_HIP_DELTA_Z: L.z = m; break;
        case Q3X_HIP_DELTA_A: L.a = m; break;
        case Q3X_HIP_DELTA_B: L.b = m; break;
        case Q3X_HIP_DELTA_CONV: L.conv = bf; break;
        case Q3X_HIP_DELTA_ALOG: L.alog = f32; break;
        case Q3X_HIP_DELTA_DT: L.dt = bf; break;
        case Q3X_HIP_DELTA_NORM: L.norm = f32; break;
        case Q3X_HIP_DELTA_OUT: L.out = m; break;
        case Q3X_HIP_ATTN_Q: L.q = m; L.attention = true; break;
        case Q3X_HIP_ATTN_K: L.k = m; break;
        case Q3X_HIP_ATTN_V: L.v = m; break;
        case Q3X_HIP_ATTN_QNORM: L.qnorm = bf; break;
        case Q3X_HIP_ATTN_KNORM: L.knorm = bf; break;
        case Q3X_HIP_ATTN_OUT: L.o = m; break;
        case Q3X_HIP_FFN_GATE: L.gate = m; break;
        case Q3X_HIP_FFN_UP: L.up = m; break;
        case Q3X_HIP_FFN_DOWN: L.down = m; break;
        case Q3X_HIP_MOE_ROUTER: L.moe.router = p; break;
        case Q3X_HIP_MOE_GATE_UP: L.moe.gate_up = p; break;
        case Q3X_HIP_MOE_DOWN: L.moe.down = p; break;
        case Q3X_HIP_MOE_SHARED_GATE: L.moe.shared_gate = p; break;
        case Q3X_HIP_MOE_SHARED_UP: L.moe.shared_up = p; break;
        case Q3X_HIP_MOE_SHARED_DOWN: L.moe.shared_down = p; break;
        case Q3X_HIP_MOE_SHARED_SCALE: L.moe.shared_scale = p; break;
        default: break;
        }
    }
    if (c.tied_embeddings) e->lm_head = e->embedding;  // engine.cpp:500
    for (auto& L : e->layers)
        L.moe = q3x_hip_moe_layer_weights{L.moe.router, L.moe.gate_up, L.moe.down, L.moe.shared_gate,
                                          L.moe.shared_up, L.moe.shared_down, L.moe.shared_scale, c.matrix_type,
                                          c.experts, c.top_k, c.H, c.I, c.shared_I};
    const int DQK = c.KH * c.KD, DO = c.VH * c.VD, DQKV = 2 * DQK + DO;
    const int AS = c.AH * c.AD, KVW = c.KVH * c.AD;
    const size_t conv = static_cast<size_t>(DQKV) * (c.CK - 1);
    const size_t memory = static_cast<size_t>(c.VH) * c.KD * c.VD;
    const size_t cache = static_cast<size_t>(context) * KVW;
    const int delta_layers = c.N - c.N / c.AI, attention_layers = c.N / c.AI;
    e->recurrent_floats = static_cast<size_t>(delta_layers) * (conv + memory);
    if (c.experts) e->moe_ws_bytes = q3x_hip_moe_layer_workspace_bytes(&e->layers[0].moe, 1);
    e->token_capacity = std::max(context, 1);
    // Arena: work vectors, recurrent state and its checkpoint, KV cache, logits.
    auto bytes = [](size_t n, size_t size) { return (n * size + 255) / 256 * 256; };
    size_t total = 0;
    const size_t work_floats[] = {static_cast<size_t>(c.H), static_cast<size_t>(c.H), static_cast<size_t>(c.H),
                                  static_cast<size_t>(c.V), static_cast<size_t>(DQKV), static_cast<size_t>(DO),
                                  static_cast<size_t>(c.VH), static_cast<size_t>(c.VH), static_cast<size_t>(DO),
                                  2 * static_cast<size_t>(AS), static_cast<size_t>(AS), static_cast<size_t>(AS),
                                  static_cast<size_t>(KVW), static_cast<size_t>(KVW), static_cast<size_t>(AS),
                                  static_cast<size_t>(c.AH) * context, static_cast<size_t>(c.I),
                                  static_cast<size_t>(c.I), e->recurrent_floats, e->recurrent_floats,
                                  static_cast<size_t>(c.V)};
    for (size_t n : work_floats) total += bytes(n, 4);
    total += static_cast<size_t>(attention_layers) * 2 * bytes(cache, 4);
    total += bytes(e->token_capacity, 4) + 3 * 256 + bytes(e->moe_ws_bytes, 1);
    int rc = Q3X_HIP_OK;
    const hipError_t status = hipMalloc(&e->arena, total);
    if (status != hipSuccess) {
        (void)hipGetLastError();
        e->arena = nullptr;
        set_error(error, "HIP engine state does not fit in device memory");
        rc = Q3X_HIP_ERUNTIME;
    }
    if (rc == Q3X_HIP_OK) {
        uint8_t* cur = static_cast<uint8_t*>(e->arena);
        e->hidden = carve<float>(cur, c.H);
        e->normalized = carve<float>(cur, c.H);
        e->branch = carve<float>(cur, c.H);
        e->logits = carve<float>(cur, c.V);
        e->qkv = carve<float>(cur, DQKV);
        e->z = carve<float>(cur, DO);
        e->a = carve<float>(cur, c.VH);
        e->b = carve<float>(cur, c.VH);
        e->delta_out = carve<float>(cur, DO);
        e->query_and_gate = carve<float>(cur, 2 * static_cast<size_t>(AS));
        e->query = carve<float>(cur, AS);
        e->gate = carve<float>(cur, AS);
        e->key = carve<float>(cur, KVW);
        e->value = carve<float>(cur, KVW);
        e->attn_out = carve<float>(cur, AS);
        e->scores = carve<float>(cur, static_cast<size_t>(c.AH) * context);
        e->ffn_gate = carve<float>(cur, c.I);
        e->ffn_up = carve<float>(cur, c.I);
        e->recurrent = carve<float>(cur, e->recurrent_floats);
        e->checkpoint_recurrent = carve<float>(cur, e->recurrent_floats);
        e->checkpoint_logits = carve<float>(cur, c.V);
        float* rec = e->recurrent;
        for (int i = 0; i < c.N; ++i) {
            LayerWeights& L = e->layers[i];
            if (!L.attention) {
                L.conv_state = rec;
                rec += conv;
                L.memory = rec;
                rec += memory;
            } else {
                L.key_cache = carve<float>(cur, cache);
                L.value_cache = carve<float>(cur, cache);
            }
        }
        e->d_tokens = carve<int>(cur, e->token_capacity);
        e->d_step = carve<int>(cur, 1);
        e->d_position = carve<int>(cur, 1);
        e->d_argmax = carve<int>(cur, 1);
        e->moe_ws = e->moe_ws_bytes ? carve<uint8_t>(cur, e->moe_ws_bytes) : nullptr;
        if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess ||
            hipHostMalloc(reinterpret_cast<void**>(&e->h_tokens), sizeof(int) * e->token_capacity,
                          hipHostMallocDefault) != hipSuccess ||
            hipMemsetAsync(e->arena, 0, total, e->stream) != hipSuccess ||
            hipStreamSynchronize(e->stream) != hipSuccess) {
            set_error(error, "HIP engine set-up failed");
            rc = Q3X_HIP_ERUNTIME;
        }
    }
    // One eager step (token 0 at position 0, then a reset) before any graph
    // capture: the launchers' once-per-process set-up (kernel attributes)
    // then happens outside a capture.
    if (rc == Q3X_HIP_OK) {
        hipLaunchKernelGGL(set_counters_kernel, dim3(1), dim3(1), 0, e->stream, e->d_step, e->d_position, 0, 0);
        rc = enqueue_step(*e, true);
        if (rc == Q3X_HIP_OK && hipStreamSynchronize(e->stream) != hipSuccess) rc = Q3X_HIP_ERUNTIME;
        if (rc == Q3X_HIP_OK) rc = q3x_hip_engine_reset(e);
        if (rc != Q3X_HIP_OK) set_error(error, "HIP engine warm-up step failed");
    }
    if (rc != Q3X_HIP_OK) {
        q3x_hip_engine_destroy(e);
        return rc;
    }
    *engine = e;
    return Q3X_HIP_OK;
}

extern "C" int q3x_hip_engine_reset(q3x_hip_engine* e) {
    if (!e) return Q3X_HIP_EINVAL;
    // engine.cpp:158-162: position 0, recurrent state zero (the KV cache is
    // overwritten before it is read).
    hipLaunchKernelGGL(set_counters_kernel, dim3(1), dim3(1), 0, e->stream, e->d_step, e->d_position, 0, 0);
    if (hipMemsetAsync(e->recurrent, 0, e->recurrent_floats * sizeof(float), e->stream) != hipSuccess ||
        hipStreamSynchronize(e->stream) != hipSuccess)
        return Q3X_HIP_ERUNTIME;
    e->position = 0;
    return Q3X_HIP_OK;
}

extern "C" int q3x_hip_engine_forward(q3x_hip_engine* e, const int* tokens, int count, int compute_logits) {
    if (!e || !tokens || count <= 0) return Q3X_HIP_EINVAL;
    if (count > e->capacity - e->position) return Q3X_HIP_EINVAL;
    for (int i = 0; i < count; ++i)
        if (tokens[i] < 0 || tokens[i] >= e->c.V) return Q3X_HIP_EINVAL;
    for (int i = 0; i < count; ++i) e->h_tokens[i] = tokens[i];
    hipLaunchKernelGGL(set_counters_kernel, dim3(1), dim3(1), 0, e->stream, e->d_step, e->d_position, 0,
                       e->position);
    if (hipMemcpyAsync(e->d_tokens, e->h_tokens, sizeof(int) * count, hipMemcpyHostToDevice, e->stream) !=
        hipSuccess)
        return Q3X_HIP_ERUNTIME;
    for (int i = 0; i < count; ++i) {
        const bool logits = compute_logits && i + 1 == count;
        hipGraphExec_t& g = e->graph[logits ? 1 : 0];
        if (!g) {
            const int rc = capture(*e, logits);
            if (rc) return rc;
        }
        if (hipGraphLaunch(g, e->stream) != hipSuccess) return Q3X_HIP_ERUNTIME;
    }
    if (hipStreamSynchronize(e->stream) != hipSuccess) return Q3X_HIP_ERUNTIME;
    e->position += count;
    return Q3X_HIP_OK;
}

extern "C" int q3x_hip_engine_logits(const q3x_hip_engine* e, float* out) {
    if (!e || !out) return Q3X_HIP_EINVAL;
    return hipMemcpy(out, e->logits, sizeof(float) * e->c.V, hipMemcpyDeviceToHost) == hipSuccess
               ? Q3X_HIP_OK
               : Q3X_HIP_ERUNTIME;
}

extern "C" int q3x_hip_engine_argmax(const q3x_hip_engine* e, int* token) {
    if (!e || !token) return Q3X_HIP_EINVAL;
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kNormThreads), 0, e->stream, e->logits, e->c.V, e->d_argmax);
    if (hipMemcpyAsync(token, e->d_argmax, sizeof(int), hipMemcpyDeviceToHost, e->stream) != hipSuccess ||
        hipStreamSynchronize(e->stream) != hipSuccess)
        return Q3X_HIP_ERUNTIME;
    return Q3X_HIP_OK;
}

extern "C" int q3x_hip_engine_checkpoint_save(q3x_hip_engine* e) {
    if (!e) return Q3X_HIP_EINVAL;
    if (hipMemcpyAsync(e->checkpoint_recurrent, e->recurrent, e->recurrent_floats * sizeof(float),
                       hipMemcpyDeviceToDevice, e->stream) != hipSuccess ||
        hipMemcpyAsync(e->checkpoint_logits, e->logits, sizeof(float) * e->c.V, hipMemcpyDeviceToDevice,
                       e->stream) != hipSuccess ||
        hipStreamSynchronize(e->stream) != hipSuccess)
        return Q3X_HIP_ERUNTIME;
    e->checkpoint_position = e->position;
    return Q3X_HIP_OK;
}

extern "C" int q3x_hip_engine_checkpoint_restore(q3x_hip_engine* e) {
    if (!e) return Q3X_HIP_EINVAL;
    if (hipMemcpyAsync(e->recurrent, e->checkpoint_recurrent, e->recurrent_floats * sizeof(float),
                       hipMemcpyDeviceToDevice, e->stream) != hipSuccess ||
        hipMemcpyAsync(e->logits, e->checkpoint_logits, sizeof(float) * e->c.V, hipMemcpyDeviceToDevice,
                       e->stream) != hipSuccess ||
        hipStreamSynchronize(e->stream) != hipSuccess)
        return Q3X_HIP_ERUNTIME;
    e->position = e->checkpoint_position;
    return Q3X_HIP_OK;
}

extern "C" int q3x_hip_engine_position(const q3x_hip_engine* e) { return e ? e->position : -1; }
