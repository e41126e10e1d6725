/*
 * q3x_oracle.c -- CPU restatement of qwen3x's quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker; see q3x_oracle.h).  The
 * product library never links this file.
 *
 * Floating-point contract: the reference is built with g++ -O3 -march=native,
 * which contracts `acc += a * b` into a single fused multiply-add.  The loops
 * below spell those FMAs out with fmaf() and the file is compiled with
 * -ffp-contract=off, so the arithmetic is the same on any x86-64 host.  The
 * equality with the reference build is checked bit for bit by the tests
 * against oracle/_ref (built from the reference sources where they lie).
 */
#include "q3x_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define Q8_BLOCK 32
#define Q8_BYTES 34 /* q8.h:10-15: uint16 scale + int8 values[32] */
#define Q4_BLOCK 32
#define Q4_BYTES 18 /* q4.h:12-15: uint16 scale + uint8 values[16] */

/* arch/cpu.cpp:31-52: exact IEEE binary16 -> binary32, subnormals included. */
float q3xo_f16(uint16_t value) {
    const uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
    uint32_t exponent = (value >> 10) & 0x1fu;
    uint32_t mantissa = value & 0x03ffu;
    uint32_t bits = 0;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            exponent = 113;
            while (!(mantissa & 0x0400u)) { mantissa <<= 1; --exponent; }
            bits = sign | (exponent << 23) | ((mantissa & 0x03ffu) << 13);
        }
    } else if (exponent == 31) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112) << 23) | (mantissa << 13);
    }
    float result;
    memcpy(&result, &bits, sizeof(result));
    return result;
}

static uint16_t load_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* q4.h:19-23: element j < 16 is the low nibble of byte j, element j >= 16 the
 * high nibble of byte j - 16; the stored nibble is biased by 8. */
static int q4_value(const uint8_t* block, int index) {
    const uint8_t packed = block[2 + index % 16];
    const int quant = index < 16 ? (packed & 0x0f) : (packed >> 4);
    return quant - 8;
}

/* arch/cpu.cpp:161-179 */
int q3xo_quantized_bytes(uint32_t type, int rows, int cols, size_t* bytes) {
    int block_size;
    size_t block_bytes;
    switch (type) {
    case Q3XO_Q8_0: block_size = Q8_BLOCK; block_bytes = Q8_BYTES; break;
    case Q3XO_Q4_0: block_size = Q4_BLOCK; block_bytes = Q4_BYTES; break;
    default: return 0;
    }
    if (rows <= 0 || cols <= 0 || cols % block_size != 0) return 0;
    const size_t blocks = (size_t)cols / block_size;
    const size_t maximum = SIZE_MAX;
    if (blocks > maximum / block_bytes) return 0;
    const size_t row_bytes = blocks * block_bytes;
    if ((size_t)rows > maximum / row_bytes) return 0;
    *bytes = (size_t)rows * row_bytes;
    return 1;
}

/* arch/cpu.cpp:55-63 (Q8_0) and 81-90 (Q4_0): out[i] = f16(d) * q_i. */
int q3xo_embed(const void* weights, uint32_t type, int cols, int row, float* out) {
    const uint8_t* w = (const uint8_t*)weights;
    if (type == Q3XO_Q8_0) {
        const int blocks = cols / Q8_BLOCK;
        const uint8_t* r = w + (size_t)row * blocks * Q8_BYTES;
        for (int block = 0; block < blocks; ++block) {
            const uint8_t* b = r + (size_t)block * Q8_BYTES;
            const float scale = q3xo_f16(load_u16(b));
            for (int i = 0; i < Q8_BLOCK; ++i)
                out[block * Q8_BLOCK + i] = scale * (float)(int8_t)b[2 + i];
        }
        return 1;
    }
    if (type == Q3XO_Q4_0) {
        const int blocks = cols / Q4_BLOCK;
        const uint8_t* r = w + (size_t)row * blocks * Q4_BYTES;
        for (int block = 0; block < blocks; ++block) {
            const uint8_t* b = r + (size_t)block * Q4_BYTES;
            const float scale = q3xo_f16(load_u16(b));
            for (int i = 0; i < Q4_BLOCK; ++i)
                out[block * Q4_BLOCK + i] = scale * (float)q4_value(b, i);
        }
        return 1;
    }
    return 0;
}

/* arch/cpu.cpp:64-73: inner = sum_i q_i x_i in order, then sum += f16(d) inner. */
static float dot_q8_0(const uint8_t* blocks, const float* x, int n) {
    float sum = 0.0f;
    for (int block = 0; block < n / Q8_BLOCK; ++block) {
        const uint8_t* b = blocks + (size_t)block * Q8_BYTES;
        float inner = 0.0f;
        for (int i = 0; i < Q8_BLOCK; ++i)
            inner = fmaf((float)(int8_t)b[2 + i], x[block * Q8_BLOCK + i], inner);
        sum = fmaf(q3xo_f16(load_u16(b)), inner, sum);
    }
    return sum;
}

/* arch/cpu.cpp:91-101 */
static float dot_q4_0(const uint8_t* blocks, const float* x, int n) {
    float sum = 0.0f;
    for (int block = 0; block < n / Q4_BLOCK; ++block) {
        const uint8_t* b = blocks + (size_t)block * Q4_BYTES;
        float inner = 0.0f;
        for (int i = 0; i < Q4_BLOCK; ++i)
            inner = fmaf((float)q4_value(b, i), x[block * Q4_BLOCK + i], inner);
        sum = fmaf(q3xo_f16(load_u16(b)), inner, sum);
    }
    return sum;
}

/* arch/cpu.cpp:74-78 and 102-106, restricted to rows [row0, row1). */
int q3xo_mv_rows(const void* weights, uint32_t type, int row0, int row1, int cols,
                 const float* x, float* y) {
    const uint8_t* w = (const uint8_t*)weights;
    if (type == Q3XO_Q8_0) {
        const size_t row_bytes = (size_t)(cols / Q8_BLOCK) * Q8_BYTES;
        for (int row = row0; row < row1; ++row)
            y[row] = dot_q8_0(w + (size_t)row * row_bytes, x, cols);
        return 1;
    }
    if (type == Q3XO_Q4_0) {
        const size_t row_bytes = (size_t)(cols / Q4_BLOCK) * Q4_BYTES;
        for (int row = row0; row < row1; ++row)
            y[row] = dot_q4_0(w + (size_t)row * row_bytes, x, cols);
        return 1;
    }
    return 0;
}

/* ---- row-parallel driver: each thread owns a disjoint row range, so the
 * result is bit-identical to the serial loop. ---- */

typedef struct {
    const void* w; uint32_t type; int cols;
    const float* X; float* Y; int rows; int count;
    long long begin, end; /* flattened (token, row) work range */
} mv_job;

static void* mv_worker(void* arg) {
    mv_job* job = (mv_job*)arg;
    long long index = job->begin;
    while (index < job->end) {
        const int token = (int)(index / job->rows);
        const int row = (int)(index % job->rows);
        long long stop = (long long)(token + 1) * job->rows;
        if (stop > job->end) stop = job->end;
        const int row_end = (int)(stop - (long long)token * job->rows);
        q3xo_mv_rows(job->w, job->type, row, row_end, job->cols,
                     job->X + (size_t)token * job->cols,
                     job->Y + (size_t)token * job->rows);
        index = stop;
    }
    return NULL;
}

int q3xo_gemm(const void* weights, uint32_t type, int rows, int cols,
              const float* X, int count, float* Y, int threads) {
    size_t bytes;
    if (!q3xo_quantized_bytes(type, rows, cols, &bytes) || count <= 0) return 0;
    if (threads < 1) threads = 1;
    const long long total = (long long)rows * count;
    if (threads > total) threads = (int)total;
    mv_job jobs[256];
    pthread_t tids[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; ++t) {
        jobs[t].w = weights; jobs[t].type = type; jobs[t].cols = cols;
        jobs[t].X = X; jobs[t].Y = Y; jobs[t].rows = rows; jobs[t].count = count;
        jobs[t].begin = total * t / threads;
        jobs[t].end = total * (t + 1) / threads;
    }
    if (threads == 1) { mv_worker(&jobs[0]); return 1; }
    for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, mv_worker, &jobs[t]);
    for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    return 1;
}

int q3xo_mv(const void* weights, uint32_t type, int rows, int cols,
            const float* x, float* y, int threads) {
    return q3xo_gemm(weights, type, rows, cols, x, 1, y, threads);
}

/* engine.cpp:187-191 */
float q3xo_sigmoid(float x) {
    if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
    const float e = expf(x);
    return e / (1.0f + e);
}
float q3xo_silu(float x) { return x * q3xo_sigmoid(x); }

/* engine.cpp:377-405: max-subtracted softmax, then top_k sequential argmax
 * passes with a strict '>' (lowest index wins ties), then renormalise. */
int q3xo_router_top_k(const float* logits, int experts, int top_k, int* ids,
                      float* weights, float* probabilities) {
    if (!(experts > 0 && top_k > 0 && top_k <= experts)) return 0;
    float maximum = -INFINITY;
    for (int e = 0; e < experts; ++e)
        maximum = maximum < logits[e] ? logits[e] : maximum; /* std::max(a, b) */
    float total = 0.0f;
    for (int e = 0; e < experts; ++e) {
        probabilities[e] = expf(logits[e] - maximum);
        total += probabilities[e];
    }
    for (int e = 0; e < experts; ++e) probabilities[e] /= total;
    float selected_total = 0.0f;
    for (int slot = 0; slot < top_k; ++slot) {
        int selected = -1;
        for (int e = 0; e < experts; ++e) {
            int used = 0;
            for (int previous = 0; previous < slot; ++previous)
                used = used || ids[previous] == e;
            if (!used && (selected < 0 || probabilities[e] > probabilities[selected]))
                selected = e;
        }
        if (selected < 0) return 0;
        ids[slot] = selected;
        selected_total += probabilities[selected];
    }
    for (int slot = 0; slot < top_k; ++slot)
        weights[slot] = probabilities[ids[slot]] / selected_total;
    return 1;
}

/* ---- routed experts: engine.cpp:406-420 with expert_mv engine.cpp:214-224 ---- */

typedef struct {
    const uint8_t* gate_up; const uint8_t* down; uint32_t type;
    int experts, H, I, top_k;
    const float* X; const int* ids; const float* weights; float* Y;
    size_t gate_up_stride, down_stride;
    int t0, t1; int ok;
} moe_job;

static void* moe_worker(void* arg) {
    moe_job* job = (moe_job*)arg;
    const int H = job->H, I = job->I;
    float* gate_up = (float*)malloc(sizeof(float) * (size_t)(2 * I + H));
    if (!gate_up) { job->ok = 0; return NULL; }
    float* delta = gate_up + 2 * I;
    for (int t = job->t0; t < job->t1; ++t) {
        const float* input = job->X + (size_t)t * H;
        float* out = job->Y + (size_t)t * H;
        for (int i = 0; i < H; ++i) out[i] = 0.0f;
        for (int slot = 0; slot < job->top_k; ++slot) {
            const int expert = job->ids[(size_t)t * job->top_k + slot];
            if (expert < 0 || expert >= job->experts) { job->ok = 0; break; }
            q3xo_mv_rows(job->gate_up + (size_t)expert * job->gate_up_stride, job->type,
                         0, 2 * I, H, input, gate_up);
            for (int i = 0; i < I; ++i)
                gate_up[i] = q3xo_silu(gate_up[i]) * gate_up[I + i];
            q3xo_mv_rows(job->down + (size_t)expert * job->down_stride, job->type,
                         0, H, I, gate_up, delta);
            const float weight = job->weights[(size_t)t * job->top_k + slot];
            for (int i = 0; i < H; ++i) out[i] = fmaf(weight, delta[i], out[i]);
        }
    }
    free(gate_up);
    return NULL;
}

int q3xo_moe_routed(const void* gate_up, const void* down, uint32_t type,
                    int experts, int H, int I, const float* X, int tokens,
                    const int* ids, const float* weights, int top_k, float* Y,
                    int threads) {
    size_t gu_bytes, down_bytes;
    if (experts <= 0 || tokens <= 0 || top_k <= 0 || top_k > experts) return 0;
    if (!q3xo_quantized_bytes(type, 2 * I, H, &gu_bytes)) return 0;
    if (!q3xo_quantized_bytes(type, H, I, &down_bytes)) return 0;
    if (threads < 1) threads = 1;
    if (threads > tokens) threads = tokens;
    if (threads > 256) threads = 256;
    moe_job jobs[256];
    pthread_t tids[256];
    for (int t = 0; t < threads; ++t) {
        moe_job* j = &jobs[t];
        j->gate_up = (const uint8_t*)gate_up; j->down = (const uint8_t*)down; j->type = type;
        j->experts = experts; j->H = H; j->I = I; j->top_k = top_k;
        j->X = X; j->ids = ids; j->weights = weights; j->Y = Y;
        j->gate_up_stride = gu_bytes; j->down_stride = down_bytes;
        j->t0 = (int)((long long)tokens * t / threads);
        j->t1 = (int)((long long)tokens * (t + 1) / threads);
        j->ok = 1;
    }
    if (threads == 1) {
        moe_worker(&jobs[0]);
    } else {
        for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, moe_worker, &jobs[t]);
        for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    }
    for (int t = 0; t < threads; ++t) if (!jobs[t].ok) return 0;
    return 1;
}

/* ---- the BF16 matvec and the whole MoE layer ---- */

/* engine.cpp:181-185 */
static float bf16_value(uint16_t value) {
    const uint32_t bits = (uint32_t)value << 16;
    float result;
    memcpy(&result, &bits, sizeof(result));
    return result;
}

/* engine.cpp:200-205: sum += f32(a) * b, contracted to an FMA by the build. */
static float dot_bf16_scalar(const uint16_t* a, const float* b, int n) {
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) sum = fmaf(bf16_value(a[i]), b[i], sum);
    return sum;
}

/* arch/x86/kernels.h:21-37, the BF16 dot a reference built with AVX-512 F and
 * BW takes (arch/cpu.cpp:112-114, 202): lane j of a 16-wide vector
 * accumulates fma(w[i], x[i]) for i = j mod 16 in element order; the lanes
 * are reduced as GCC's _mm512_reduce_add_ps does (upper 8 + lower 8, upper 4
 * + lower 4, then elements 0 + 2 and 1 + 3, then those two); the tail past
 * the last 16 adds sum = fma(w[i], x[i], sum) in order. */
static float dot_bf16_x16(const uint16_t* a, const float* b, int n) {
    float lane[16] = {0};
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; ++j) lane[j] = fmaf(bf16_value(a[i + j]), b[i + j], lane[j]);
    float t3[8], t6[4];
    for (int j = 0; j < 8; ++j) t3[j] = lane[8 + j] + lane[j];
    for (int j = 0; j < 4; ++j) t6[j] = t3[4 + j] + t3[j];
    const float t8_0 = t6[0] + t6[2], t8_1 = t6[1] + t6[3];
    float sum = t8_0 + t8_1;
    for (; i < n; ++i) sum = fmaf(bf16_value(a[i]), b[i], sum);
    return sum;
}

/* Which BF16 dot the reference build in use takes: 1 (portable scalar loop)
 * or 16 (AVX-512). */
static int bf16_lanes = 1;

int q3xo_set_bf16_lanes(int lanes) {
    if (lanes != 1 && lanes != 16) return 0;
    bf16_lanes = lanes;
    return 1;
}

static float dot_bf16(const uint16_t* a, const float* b, int n) {
    return bf16_lanes == 16 ? dot_bf16_x16(a, b, n) : dot_bf16_scalar(a, b, n);
}

/* engine.cpp:207-212 (the BF16 branch of mv) */
int q3xo_mv_bf16(const uint16_t* weights, int rows, int cols, const float* x, float* y) {
    if (rows <= 0 || cols <= 0) return 0;
    for (int r = 0; r < rows; ++r) y[r] = dot_bf16(weights + (size_t)r * cols, x, cols);
    return 1;
}

typedef struct {
    const uint16_t* router; const uint8_t* gate_up; const uint8_t* down;
    const uint8_t* shared_gate; const uint8_t* shared_up; const uint8_t* shared_down;
    const uint16_t* shared_scale; uint32_t type;
    int experts, H, I, shared_I, top_k;
    const float* X; float* Y; int* ids; float* weights;
    size_t gate_up_stride, down_stride;
    int t0, t1; int ok;
} layer_job;

/* engine.cpp:406-430 for tokens [t0, t1). */
static void* layer_worker(void* arg) {
    layer_job* job = (layer_job*)arg;
    const int H = job->H, I = job->I, SI = job->shared_I, E = job->experts, K = job->top_k;
    /* logits, probabilities, gate_up (2I), delta (H) */
    float* logits = (float*)malloc(sizeof(float) * ((size_t)2 * E + 2 * I + H));
    if (!logits) { job->ok = 0; return NULL; }
    float* probabilities = logits + E;
    float* gate_up = probabilities + E;
    float* delta = gate_up + 2 * I;
    int ids[64];
    float weights[64];
    for (int t = job->t0; t < job->t1 && job->ok; ++t) {
        const float* input = job->X + (size_t)t * H;
        float* out = job->Y + (size_t)t * H;
        q3xo_mv_bf16(job->router, E, H, input, logits);                       /* :408 */
        if (!q3xo_router_top_k(logits, E, K, ids, weights, probabilities)) {  /* :409 */
            job->ok = 0;
            break;
        }
        for (int i = 0; i < H; ++i) out[i] = 0.0f;                            /* :411 */
        for (int slot = 0; slot < K; ++slot) {                                /* :412-420 */
            const int expert = ids[slot];
            q3xo_mv_rows(job->gate_up + (size_t)expert * job->gate_up_stride, job->type, 0, 2 * I, H,
                         input, gate_up);
            for (int i = 0; i < I; ++i) gate_up[i] = q3xo_silu(gate_up[i]) * gate_up[I + i];
            q3xo_mv_rows(job->down + (size_t)expert * job->down_stride, job->type, 0, H, I, gate_up, delta);
            for (int i = 0; i < H; ++i) out[i] = fmaf(weights[slot], delta[i], out[i]);
        }
        /* :422-429: gate into gate_up[0, SI), up into gate_up[I, I + SI) */
        q3xo_mv_rows(job->shared_gate, job->type, 0, SI, H, input, gate_up);
        q3xo_mv_rows(job->shared_up, job->type, 0, SI, H, input, gate_up + I);
        for (int i = 0; i < SI; ++i) gate_up[i] = q3xo_silu(gate_up[i]) * gate_up[I + i];
        q3xo_mv_rows(job->shared_down, job->type, 0, H, SI, gate_up, delta);
        const float scale = q3xo_sigmoid(dot_bf16(job->shared_scale, input, H));
        for (int i = 0; i < H; ++i) out[i] = fmaf(scale, delta[i], out[i]);
        for (int slot = 0; slot < K; ++slot) {
            if (job->ids) job->ids[(size_t)t * K + slot] = ids[slot];
            if (job->weights) job->weights[(size_t)t * K + slot] = weights[slot];
        }
    }
    free(logits);
    return NULL;
}

int q3xo_moe_layer(const uint16_t* router, const void* gate_up, const void* down,
                   const void* shared_gate, const void* shared_up, const void* shared_down,
                   const uint16_t* shared_scale, uint32_t type, int experts, int H, int I,
                   int shared_I, int top_k, const float* X, int tokens, float* Y, int* ids,
                   float* weights, int threads) {
    size_t gu_bytes, down_bytes, sg_bytes, sd_bytes;
    if (experts <= 0 || tokens <= 0 || top_k <= 0 || top_k > experts || top_k > 64) return 0;
    if (shared_I <= 0 || shared_I > I) return 0;
    if (!q3xo_quantized_bytes(type, 2 * I, H, &gu_bytes)) return 0;
    if (!q3xo_quantized_bytes(type, H, I, &down_bytes)) return 0;
    if (!q3xo_quantized_bytes(type, shared_I, H, &sg_bytes)) return 0;
    if (!q3xo_quantized_bytes(type, H, shared_I, &sd_bytes)) return 0;
    if (threads < 1) threads = 1;
    if (threads > tokens) threads = tokens;
    if (threads > 256) threads = 256;
    layer_job jobs[256];
    pthread_t tids[256];
    for (int t = 0; t < threads; ++t) {
        layer_job* j = &jobs[t];
        j->router = router; j->gate_up = (const uint8_t*)gate_up; j->down = (const uint8_t*)down;
        j->shared_gate = (const uint8_t*)shared_gate; j->shared_up = (const uint8_t*)shared_up;
        j->shared_down = (const uint8_t*)shared_down; j->shared_scale = shared_scale; j->type = type;
        j->experts = experts; j->H = H; j->I = I; j->shared_I = shared_I; j->top_k = top_k;
        j->X = X; j->Y = Y; j->ids = ids; j->weights = weights;
        j->gate_up_stride = gu_bytes; j->down_stride = down_bytes;
        j->t0 = (int)((long long)tokens * t / threads);
        j->t1 = (int)((long long)tokens * (t + 1) / threads);
        j->ok = 1;
    }
    if (threads == 1) {
        layer_worker(&jobs[0]);
    } else {
        for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, layer_worker, &jobs[t]);
        for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    }
    for (int t = 0; t < threads; ++t) if (!jobs[t].ok) return 0;
    return 1;
}

/* ---- scripts/pack_weights.py:299-343 quantizers on float32 values ---- */

/* numpy float32 -> float16 cast: IEEE round-to-nearest-even, overflow to inf. */
static uint16_t f32_to_f16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, sizeof(bits));
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t exponent = (bits >> 23) & 0xffu;
    uint32_t mantissa = bits & 0x7fffffu;
    if (exponent == 0xff) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (mantissa ? 0x200u | (mantissa >> 13) : 0u));
    const int e = (int)exponent - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) { /* subnormal half (or zero) */
        if (e < -10) return sign;
        mantissa |= 0x800000u;
        const int shift = 14 - e; /* 14..24 */
        uint32_t half = mantissa >> shift;
        const uint32_t rest = mantissa & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1);
        if (rest > halfway || (rest == halfway && (half & 1u))) ++half;
        return (uint16_t)(sign | half);
    }
    uint32_t half = ((uint32_t)e << 10) | (mantissa >> 13);
    const uint32_t rest = mantissa & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (half & 1u))) ++half; /* may carry into inf */
    return (uint16_t)(sign | half);
}

int q3xo_quantize(uint32_t type, const float* values, size_t n, void* out) {
    if (n % 32) return 0;
    for (size_t i = 0; i < n; ++i) if (!isfinite(values[i])) return 0;
    uint8_t* o = (uint8_t*)out;
    const size_t blocks = n / 32;
    for (size_t block = 0; block < blocks; ++block) {
        const float* v = values + block * 32;
        if (type == Q3XO_Q8_0) {
            float maximum = 0.0f; /* np.max(np.abs(values)) */
            for (int i = 0; i < 32; ++i) { const float a = fabsf(v[i]); if (a > maximum) maximum = a; }
            const float scale = maximum / 127.0f;
            const float inverse = scale != 0.0f ? 1.0f / scale : 0.0f;
            uint8_t* b = o + block * Q8_BYTES;
            const uint16_t h = f32_to_f16(scale);
            b[0] = (uint8_t)(h & 0xff); b[1] = (uint8_t)(h >> 8);
            for (int i = 0; i < 32; ++i) {
                const float normalized = v[i] * inverse;
                float rounded = copysignf(floorf(fabsf(normalized) + 0.5f), normalized);
                if (rounded > 127.0f) rounded = 127.0f;
                if (rounded < -127.0f) rounded = -127.0f;
                b[2 + i] = (uint8_t)(int8_t)(int)rounded;
            }
        } else if (type == Q3XO_Q4_0) {
            int largest = 0; /* np.argmax(np.abs(values)): first maximum wins */
            for (int i = 1; i < 32; ++i) if (fabsf(v[i]) > fabsf(v[largest])) largest = i;
            const float maximum = v[largest];
            const float scale = maximum / -8.0f;
            const float inverse = scale != 0.0f ? 1.0f / scale : 0.0f;
            uint8_t quants[32];
            for (int i = 0; i < 32; ++i) {
                float q = truncf(v[i] * inverse + 8.5f);
                if (q > 15.0f) q = 15.0f;
                quants[i] = (uint8_t)(int)q;
            }
            uint8_t* b = o + block * Q4_BYTES;
            const uint16_t h = f32_to_f16(scale);
            b[0] = (uint8_t)(h & 0xff); b[1] = (uint8_t)(h >> 8);
            for (int i = 0; i < 16; ++i) b[2 + i] = (uint8_t)(quants[i] | (quants[16 + i] << 4));
        } else {
            return 0;
        }
    }
    return 1;
}
