// engine.hip -- the decode engine: tokens through every layer of a Q8_0 /
// Q4_0 Qwen3.5 / 3.6 / 3.8 model on the GPU, the caller of the matmul path.
//
// Follows the reference's forward (engine.cpp:431-454) layer for layer:
// embedding; per layer RMSNorm, the mixer (gated DeltaNet, engine.cpp:
// 274-316, or full attention, :318-362), residual, RMSNorm, FFN or MoE,
// residual; final RMSNorm and lm_head.  A decode step runs each projection
// group (and lm_head) as one launch of the pipelined matvec (matvec.h) whose
// input staging forms the preceding RMSNorm or SwiGLU on the way into LDS
// (NormInput in matvec.h, SwiGLUInput below); output projections and down
// accumulate into the residual, and an MoE layer normalises the residual
// inside its own launches and adds its output to it directly (moe.h).  A chunk goes through this library's own entry points
// (q3x_hip_gemm, q3x_hip_moe_layer).  The kernels here are the per-token
// operations between the matrices.
//
// Every buffer lives on the device for the life of the engine: the work
// rows, the DeltaNet recurrent state (conv history and the KD x VD memory of
// each head), the KV cache, the logits.  The tokens and the position are
// read from device memory, so one decode step is position-independent and
// is captured once into a hipGraph (two: with and without logits) and
// replayed for every token, as the reference captures its step
// (arch/cuda/engine.cu:1995-2005).  A forward of several tokens runs them
// as chunks of up to kChunk rows: the matrices as prefill GEMMs
// (q3x_hip_gemm, q3x_hip_moe_layer's grouped path), the conv over runs of
// tokens and the delta-rule recurrence token by token with the state in
// registers, norms, RoPE and attention (FP32 MFMA) over all rows at once --
// the role of the reference's prefill_chunk_* (arch/cuda/engine.cu:
// 1881-1960).
#include <math.h>

#include <algorithm>
#include <new>
#include <type_traits>
#include <vector>

#include "common.h"
#include "matvec.h"
#include "moe.h"
#include "rows.h"

struct q3x_hip_engine;

namespace q3x {
namespace {

constexpr float kTheta = 10000000.0f;   // engine.cpp:26 THETA
constexpr int kNormThreads = 1024;
constexpr int kHeadThreads = 256;

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

// Rows of the embedding for tokens tokens[*step + r], r = blockIdx.y,
// dequantised bit for bit as the reference's embed (engine.cpp:195-200 via
// arch/cpu.cpp:55-63, 81-90).
template <uint32_t QT>
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t* __restrict__ w, int cols,
                                                    const int* __restrict__ tokens, const int* __restrict__ step,
                                                    float* __restrict__ out) {
    constexpr int BB = QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : kQ4Bytes;
    const int r = blockIdx.y;
    const int token = tokens[*step + r];
    const int bpr = cols / kBlock;
    const uint8_t* row = w + static_cast<size_t>(token) * bpr * BB;
    float* o = out + static_cast<size_t>(r) * cols;
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
        o[c] = scale * static_cast<float>(q);
    }
}

// Row r = blockIdx.x: out = RMSNorm(hidden) * (1 + w) (engine.cpp:228-233);
// with `branch`, hidden += branch first and is written back (the residual
// add of engine.cpp:240-242 that precedes the norm).
__global__ __launch_bounds__(kNormThreads) void rms_kernel(float* __restrict__ hidden, const float* __restrict__ branch,
                                                           const uint16_t* __restrict__ w, int n,
                                                           float* __restrict__ out) {
    __shared__ float partial[kNormThreads / kWave];
    const size_t base = static_cast<size_t>(blockIdx.x) * n;
    float* x = hidden + base;
    float square = 0.0f;
    for (int i = threadIdx.x; i < n; i += kNormThreads) {
        float v = x[i];
        if (branch) {
            v += branch[base + i];
            x[i] = v;
        }
        square = fmaf(v, v, square);
    }
    const float total = block_sum<kNormThreads>(square, partial);
    const float scale = 1.0f / sqrtf(total / static_cast<float>(n) + kEps);
    for (int i = threadIdx.x; i < n; i += kNormThreads) out[base + i] = x[i] * scale * (1.0f + bf16_value(w[i]));
}

// Causal depthwise convolution over the DQKV channels with CK - 1
// remembered inputs, then SiLU (engine.cpp:251-261), for `count` tokens
// (rows of qkv, in place).  A workgroup holds kConvChannels channels, each
// cut into kConvSegments runs of consecutive tokens, one thread per run with
// its window in registers.  Every thread first reads the CK - 1 raw inputs
// before its run (the previous run's last rows, or the remembered history for
// the first tokens); after one barrier the runs are convolved in place and
// the thread holding the last token leaves the last CK - 1 raw inputs as the
// new history.  The arithmetic per token is the reference's (conv_apply).
// The history is kept in two copies, [2][channels][CK - 1]: a forward at
// position p reads copy p % 2 and leaves copy (p + count) % 2, so a decode
// step (delta_step_kernel, which convolves its own channels) can read the
// old history of a channel that another workgroup is updating.  SEGMENTS: 16
// runs per channel.
constexpr int kMaxConv = 8;
constexpr int kConvThreads = 256;
template <int SEGMENTS>
__global__ __launch_bounds__(kConvThreads) void delta_conv_kernel(float* __restrict__ qkv,
                                                                  const uint16_t* __restrict__ w,
                                                                  float* __restrict__ history,
                                                                  const int* __restrict__ position, int channels,
                                                                  int CK, int count) {
    constexpr int kChannels = kConvThreads / SEGMENTS;
    const int c = blockIdx.x * kChannels + threadIdx.x % kChannels;
    const int segment = threadIdx.x / kChannels;
    const bool ok = c < channels;
    const int per = (count + SEGMENTS - 1) / SEGMENTS;
    const int t0 = min(count, segment * per), t1 = min(count, t0 + per);
    const int p0 = *position;
    const size_t copy = static_cast<size_t>(channels) * (CK - 1);
    const float* hist = history + (p0 & 1) * copy + static_cast<size_t>(ok ? c : 0) * (CK - 1);
    float* hist_out = history + ((p0 + count) & 1) * copy + static_cast<size_t>(ok ? c : 0) * (CK - 1);
    float past[kMaxConv - 1], wt[kMaxConv];
#pragma unroll
    for (int i = 0; i < kMaxConv; ++i) wt[i] = ok && i < CK ? bf16_value(w[static_cast<size_t>(c) * CK + i]) : 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxConv - 1; ++i) {
        const int tt = t0 - (CK - 1) + i;  // the raw input i places before the run's first token
        past[i] = !ok || i >= CK - 1 ? 0.0f : tt >= 0 ? qkv[static_cast<size_t>(tt) * channels + c] : hist[tt + CK - 1];
    }
    __syncthreads();  // every raw input and history read precedes the writes
    if (!ok) return;
    float last = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxConv; ++i)
        if (i == CK - 1) last = wt[i];
    // The run in batches of kAhead tokens, the next batch's inputs requested
    // before the current batch is convolved (its rows are this run's own and
    // not yet written), so one batch's loads are in flight while another
    // computes.
    constexpr int kAhead = 8;
    float xs[kAhead], xn[kAhead];
    auto fetch = [&](int b, float (&dst)[kAhead]) {
#pragma unroll
        for (int u = 0; u < kAhead; ++u) dst[u] = b + u < t1 ? qkv[static_cast<size_t>(b + u) * channels + c] : 0.0f;
    };
    fetch(t0, xs);
    for (int b = t0; b < t1; b += kAhead) {
        fetch(b + kAhead, xn);
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {
            if (b + u >= t1) break;
            const float x = xs[u];
            float sum = x * last;
#pragma unroll
            for (int i = 0; i < kMaxConv - 1; ++i)
                if (i < CK - 1) sum = fmaf(past[i], wt[i], sum);
#pragma unroll
            for (int i = 0; i < kMaxConv - 2; ++i)
                if (i < CK - 2) past[i] = past[i + 1];
#pragma unroll
            for (int i = 0; i < kMaxConv - 1; ++i)
                if (i == CK - 2) past[i] = x;
            qkv[static_cast<size_t>(b + u) * channels + c] = silu_ref(sum);
        }
#pragma unroll
        for (int u = 0; u < kAhead; ++u) xs[u] = xn[u];
    }
    if (t0 < t1 && t1 == count) {
#pragma unroll
        for (int i = 0; i < kMaxConv - 1; ++i)
            if (i < CK - 1) hist_out[i] = past[i];
    }
}

// One token of the causal conv of one channel, then SiLU (the arithmetic of
// delta_conv_kernel: sum = x * w[CK - 1], then sum = fma(past[i], w[i], sum)
// for the CK - 1 remembered inputs, weights BF16), in two halves so that a
// decode step can request every input before it knows the position:
// conv_fetch loads the channel's input, both history copies and the
// weights; conv_apply picks the copy by position parity, convolves, and
// leaves the shifted history in `hist_out` if not null.
struct ConvInputs {
    float x;
    float past[2][kMaxConv - 1];
    float w[kMaxConv];
};
__device__ __forceinline__ void conv_fetch(ConvInputs& in, float x, const float* history, size_t copy,
                                           const uint16_t* w, int ci, int CK) {
    in.x = x;
    const float* h0 = history + static_cast<size_t>(ci) * (CK - 1);
#pragma unroll
    for (int i = 0; i < kMaxConv - 1; ++i) {
        in.past[0][i] = i < CK - 1 ? h0[i] : 0.0f;
        in.past[1][i] = i < CK - 1 ? h0[copy + i] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kMaxConv; ++i) in.w[i] = i < CK ? bf16_value(w[static_cast<size_t>(ci) * CK + i]) : 0.0f;
}
__device__ __forceinline__ float conv_apply(const ConvInputs& in, int parity, int CK, float* hist_out) {
    float past[kMaxConv - 1];
#pragma unroll
    for (int i = 0; i < kMaxConv - 1; ++i) past[i] = parity ? in.past[1][i] : in.past[0][i];
    float last = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxConv; ++i)
        if (i == CK - 1) last = in.w[i];
    float sum = in.x * last;
#pragma unroll
    for (int i = 0; i < kMaxConv - 1; ++i)
        if (i < CK - 1) sum = fmaf(past[i], in.w[i], sum);
    if (hist_out) {
#pragma unroll
        for (int i = 0; i < kMaxConv - 1; ++i)
            if (i < CK - 1) hist_out[i] = i + 1 < CK - 1 ? past[i + 1] : in.x;
    }
    return silu_ref(sum);
}

// The DeltaNet memory S of a value head is stored column by column,
// S[c * KD + k] (value column c, key k), so a thread's run of consecutive
// keys of one column is contiguous: 16-byte accesses when KD % 4 == 0.
template <int N>
__device__ __forceinline__ void load_keys(const float* col, int k0, int KD, bool ok, float* s) {
    if (ok && KD % 4 == 0 && k0 + N <= KD) {
#pragma unroll
        for (int j = 0; j < N; j += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(col + k0 + j);
            s[j] = v.x; s[j + 1] = v.y; s[j + 2] = v.z; s[j + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) s[j] = ok && k0 + j < KD ? col[k0 + j] : 0.0f;
    }
}
template <int N>
__device__ __forceinline__ void store_keys(float* col, int k0, int KD, bool ok, const float* s) {
    if (ok && KD % 4 == 0 && k0 + N <= KD) {
#pragma unroll
        for (int j = 0; j < N; j += 4) *reinterpret_cast<f32x4*>(col + k0 + j) = f32x4{s[j], s[j + 1], s[j + 2], s[j + 3]};
    } else if (ok) {
#pragma unroll
        for (int j = 0; j < N; ++j)
            if (k0 + j < KD) col[k0 + j] = s[j];
    }
}

// Prefill form of the delta rule, in three launches so that only the
// recurrence itself runs token by token:
//   delta_prep_kernel (row r, key head kh; parallel): q, k of the head
//     L2-normalised in place (q also divided by sqrt(KD)); for the value
//     heads of kh, b <- beta = sigmoid(b) and a <- decay in place (the
//     memory is scaled by exp(decay), engine.cpp:279);
//   delta_scan_kernel (value head; sequential over the rows): the memory
//     update of the gated delta rule (engine.cpp:262-316), writing q S
//     unnormalised;
//   delta_norm_kernel (row, value head; parallel): the gated RMSNorm
//     (engine.cpp:234-239).
// A decode step runs the same arithmetic for one token (delta_step_kernel).
constexpr int kScanTile = 32;  // rows of q / k staged in LDS at a time

__global__ __launch_bounds__(128) void delta_prep_kernel(float* __restrict__ qkv, float* __restrict__ a,
                                                         float* __restrict__ b, const float* __restrict__ alog,
                                                         const uint16_t* __restrict__ dt, int KH, int VH, int KD,
                                                         int VD) {
    __shared__ float partial[128 / kWave];
    const int kh = blockIdx.x, r = blockIdx.y;
    const int t = threadIdx.x;
    const int DQK = KH * KD, DQKV = 2 * DQK + VH * VD;
    float* row = qkv + static_cast<size_t>(r) * DQKV;
    const float qv = t < KD ? row[kh * KD + t] : 0.0f;
    const float kv = t < KD ? row[DQK + kh * KD + t] : 0.0f;
    const float qn = block_sum<128>(qv * qv, partial);
    const float kn = block_sum<128>(kv * kv, partial);
    if (t < KD) {
        row[kh * KD + t] = qv * (1.0f / sqrtf(qn + kEps)) / sqrtf(static_cast<float>(KD));
        row[DQK + kh * KD + t] = kv * (1.0f / sqrtf(kn + kEps));
    }
    const int per = VH / KH;
    for (int u = t; u < per; u += 128) {
        const int head = kh * per + u;
        const size_t at = static_cast<size_t>(r) * VH + head;
        b[at] = sigmoid_ref(b[at]);
        a[at] = -expf(alog[head]) * softplus_ref(a[at] + bf16_value(dt[head]));  // decay; e^decay scales S
    }
}

// delta_scan_kernel: the value columns of a head update independently, so
// a head's 128 columns are split over kScanSlices workgroups of 4 waves
// (spreading the recurrence's arithmetic over that many CUs).  Lane l of
// wave w owns value column 32 slice + 8 w + l / 8 and keys 16 (l % 8) .. +
// 15, its S entries in registers across the tokens.  A column's eight key
// groups sit in one row half of lanes, so the sums over keys (k S before the
// update, q S after it) are three DPP adds: the tokens run with no barrier
// between them.  Per key and token: k S, the decayed update S e^decay + k
// (beta delta), and q S -- the decay multiplies k S once instead of every S
// entry before it.  q, k and the slice's v of kScanTile tokens are staged in
// LDS at a time, the next tile's loads in flight while the current one is
// processed.
constexpr int kScanThreads = 256;
constexpr int kScanCols = 32;                         // value columns per workgroup
constexpr int kScanSlices = 128 / kScanCols;          // workgroups per value head
constexpr int kScanGroups = 8;                        // key groups per column (lanes)
constexpr int kScanKeys = 128 / kScanGroups;          // keys per lane
constexpr int kScanValues = (2 * 128 + kScanCols) * kScanTile;  // staged values per tile
constexpr int kScanLoads = kScanValues / kScanThreads;          // per thread

__global__ __launch_bounds__(kScanThreads) void delta_scan_kernel(const float* __restrict__ qkv,
                                                                  const float* __restrict__ decay,
                                                                  const float* __restrict__ beta,
                                                                  float* __restrict__ memory, float* __restrict__ out,
                                                                  int KH, int VH, int KD, int VD, int count) {
    // q | k of the tile's tokens (128 slots each, zeros past KD), then the
    // slice's v (zeros past VD).
    __shared__ __attribute__((aligned(16))) float tile[kScanValues];
    __shared__ float st[kScanTile], bt[kScanTile];
    const float* const qt = tile;
    const float* const kt = tile + kScanTile * 128;
    const float* const vt = tile + 2 * kScanTile * 128;
    const int head = blockIdx.x / kScanSlices, slice = blockIdx.x % kScanSlices;
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1), wave = t / kWave;
    const int DQK = KH * KD, DO = VH * VD, DQKV = 2 * DQK + DO;
    const int kh = head / (VH / KH);
    const int cl = wave * (kWave / kScanGroups) + lane / kScanGroups;  // column within the slice
    const int c = slice * kScanCols + cl, k0 = (lane % kScanGroups) * kScanKeys;
    const bool col = c < VD;
    float* S = memory + (static_cast<size_t>(head) * VD + (col ? c : 0)) * KD;  // column c
    float s[kScanKeys];
    load_keys<kScanKeys>(S, k0, KD, col, s);
    float pre[kScanLoads], pst = 0.0f, pbt = 0.0f;
    auto load_tile = [&](int r0) {
        const int nt = min(kScanTile, count - r0);
#pragma unroll
        for (int i = 0; i < kScanLoads; ++i) {
            const int e = t + i * kScanThreads;
            float x = 0.0f;
            if (e < 2 * kScanTile * 128) {
                const int arr = e / (kScanTile * 128), rr = (e / 128) % kScanTile, k = e % 128;
                if (rr < nt && k < KD)
                    x = qkv[static_cast<size_t>(r0 + rr) * DQKV + (arr == 0 ? 0 : DQK) + kh * KD + k];
            } else {
                const int v = e - 2 * kScanTile * 128, rr = v / kScanCols, cc = slice * kScanCols + v % kScanCols;
                if (rr < nt && cc < VD) x = qkv[static_cast<size_t>(r0 + rr) * DQKV + 2 * DQK + head * VD + cc];
            }
            pre[i] = x;
        }
        if (t < nt) {
            pst = expf(decay[static_cast<size_t>(r0 + t) * VH + head]);  // e^decay
            pbt = beta[static_cast<size_t>(r0 + t) * VH + head];
        }
    };
    load_tile(0);
    for (int r0 = 0; r0 < count; r0 += kScanTile) {
        const int nt = min(kScanTile, count - r0);
        __syncthreads();  // the previous tile is consumed
#pragma unroll
        for (int i = 0; i < kScanLoads; ++i) tile[t + i * kScanThreads] = pre[i];
        if (t < kScanTile) {
            st[t] = pst;
            bt[t] = pbt;
        }
        __syncthreads();
        if (r0 + kScanTile < count) load_tile(r0 + kScanTile);
        for (int rr = 0; rr < nt; ++rr) {
            const f32x4* kp = reinterpret_cast<const f32x4*>(kt + rr * 128 + k0);
            const f32x4* qp = reinterpret_cast<const f32x4*>(qt + rr * 128 + k0);
            const float sc = st[rr], bb = bt[rr];
            const float vv = vt[rr * kScanCols + cl];
            float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
            for (int j4 = 0; j4 < kScanKeys / 4; ++j4) {
                const f32x4 kk = kp[j4];
                p0 = fmaf(kk.x, s[4 * j4 + 0], p0);
                p1 = fmaf(kk.y, s[4 * j4 + 1], p1);
                p0 = fmaf(kk.z, s[4 * j4 + 2], p0);
                p1 = fmaf(kk.w, s[4 * j4 + 3], p1);
            }
            float pred = p0 + p1;
            pred += dpp_f32<0xB1>(pred);   // the eight key groups: pairs,
            pred += dpp_f32<0x4E>(pred);   // quads,
            pred += dpp_f32<0x141>(pred);  // the two quads of the row half
            const float bd = bb * (vv - sc * pred);  // beta (v - k S e^decay)
            float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
            for (int j4 = 0; j4 < kScanKeys / 4; ++j4) {
                const f32x4 kk = kp[j4], qq = qp[j4];
                s[4 * j4 + 0] = fmaf(s[4 * j4 + 0], sc, kk.x * bd);
                s[4 * j4 + 1] = fmaf(s[4 * j4 + 1], sc, kk.y * bd);
                s[4 * j4 + 2] = fmaf(s[4 * j4 + 2], sc, kk.z * bd);
                s[4 * j4 + 3] = fmaf(s[4 * j4 + 3], sc, kk.w * bd);
                o0 = fmaf(qq.x, s[4 * j4 + 0], o0);
                o1 = fmaf(qq.y, s[4 * j4 + 1], o1);
                o0 = fmaf(qq.z, s[4 * j4 + 2], o0);
                o1 = fmaf(qq.w, s[4 * j4 + 3], o1);
            }
            float o = o0 + o1;
            o += dpp_f32<0xB1>(o);
            o += dpp_f32<0x4E>(o);
            o += dpp_f32<0x141>(o);
            if (lane % kScanGroups == 0 && col) out[static_cast<size_t>(r0 + rr) * DO + head * VD + c] = o;
        }
    }
    store_keys<kScanKeys>(S, k0, KD, col, s);
}

// The prefill recurrence in chunks of kDeltaChunk tokens on the matrix
// cores (the WY form of the gated delta rule).  With the memory S0 before a
// chunk, G_t = decay_1 + ... + decay_t inside it (so the reference's
// per-token S <- e^decay S, p = S^T k, S <- S + beta k (v - p)^T, o = S^T q,
// engine.cpp:262-316, unrolls to S_t = e^G_t S0 + sum_{j<=t} e^(G_t - G_j)
// k_j u_j^T), the updates u_t = beta_t (v_t - p_t) solve
//   (I + A) U = beta (V - e^G (K S0)),  A_tj = beta_t e^(G_t - G_j) k_t.k_j (j < t),
// so U = U0 - W S0 with U0 = (I + A)^-1 beta V and W = (I + A)^-1 beta e^G K,
// and
//   O = e^G (Q S0) + P U,   P_tj = e^(G_t - G_j) q_t.k_j (j <= t),
//   S_C = e^G_C S0 + K^T (e^(G_C - G) U).
// delta_chunk_prep_kernel forms W, U0, P, e^G, e^(G_C - G) and e^G_C of
// every (chunk, value head) in parallel (every exponent is <= 0);
// delta_chunk_scan_kernel then runs the chunks of a head in order with Q
// and K read from the projections, four FP32 MFMA products per chunk.
// Tokens past the last row are zeros in the prep (k = q = v = 0, beta = 0,
// decay 0), so their rows of W, U0 and P are zero and they change nothing.
// The sums run in another order than the reference's token loop (FP32
// throughout).
constexpr int kDeltaChunk = 32;
constexpr int kDeltaPitch = 132;  // LDS rows of K, Q, V (16-byte aligned)
constexpr int kDeltaTile = kDeltaChunk * 128;  // one [32][128] block
// Per (chunk, value head): W and U0 [32][128], P [32][32], e^G [32],
// e^(G_C - G) [32], e^G_C (padded to a multiple of 16 floats).
constexpr int kDeltaChunkFloats = 2 * kDeltaTile + kDeltaChunk * kDeltaChunk + 80;
constexpr int kDeltaPrepThreads = 256;

// Token row of register r of a 32x32 FP32 MFMA accumulator in lane half kh.
__device__ __forceinline__ int mfma32_row(int r, int kh) { return 8 * (r >> 2) + 4 * kh + (r & 3); }

// One (chunk, value head) per workgroup of 4 waves.  K K^T and Q K^T are
// two 32x32x128 products on the matrix cores (each wave one half of the
// 128 keys of one of them); the triangular solve for W and U0 runs one
// thread per column.
__global__ __launch_bounds__(kDeltaPrepThreads) void delta_chunk_prep_kernel(
    const float* __restrict__ qkv, const float* __restrict__ decay, const float* __restrict__ beta,
    float* __restrict__ ws, int KH, int VH, int KD, int VD, int count) {
    __shared__ __attribute__((aligned(16))) float kl[kDeltaChunk * kDeltaPitch];
    __shared__ __attribute__((aligned(16))) float ql[kDeltaChunk * kDeltaPitch];
    __shared__ __attribute__((aligned(16))) float vl[kDeltaChunk * kDeltaPitch];
    __shared__ float dl[kDeltaChunk], gl[kDeltaChunk], bl[kDeltaChunk], eg[kDeltaChunk];
    const int chunk = blockIdx.x, head = blockIdx.y;
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1), wave = t / kWave, li = lane & 31, kh = lane >> 5;
    const int DQK = KH * KD, DQKV = 2 * DQK + VH * VD;
    const int khead = head / (VH / KH);
    const int r0 = chunk * kDeltaChunk;
    const int n = min(kDeltaChunk, count - r0);
    float* const W = ws + (static_cast<size_t>(chunk) * VH + head) * kDeltaChunkFloats;
    float* const U0 = W + kDeltaTile;
    float* const P = W + 2 * kDeltaTile;
    float* const E = P + kDeltaChunk * kDeltaChunk;
    float* const EC = E + kDeltaChunk;
    float* const GC = EC + kDeltaChunk;
    // k, q (key head khead) and v (value head) of the chunk's rows; zeros
    // past the rows and past KD / VD.
    const f32x4 zero{0.0f, 0.0f, 0.0f, 0.0f};
    for (int e = t; e < kDeltaChunk * 32; e += kDeltaPrepThreads) {
        const int r = e / 32, c = 4 * (e % 32);
        const float* row = qkv + static_cast<size_t>(r0 + r) * DQKV;
        const bool in = r < n;
        const f32x4 kv = in && c < KD ? *reinterpret_cast<const f32x4*>(row + DQK + khead * KD + c) : zero;
        const f32x4 qv = in && c < KD ? *reinterpret_cast<const f32x4*>(row + khead * KD + c) : zero;
        const f32x4 vv = in && c < VD ? *reinterpret_cast<const f32x4*>(row + 2 * DQK + head * VD + c) : zero;
        *reinterpret_cast<f32x4*>(kl + r * kDeltaPitch + c) = kv;
        *reinterpret_cast<f32x4*>(ql + r * kDeltaPitch + c) = qv;
        *reinterpret_cast<f32x4*>(vl + r * kDeltaPitch + c) = vv;
    }
    if (t < kDeltaChunk) {
        dl[t] = t < n ? decay[static_cast<size_t>(r0 + t) * VH + head] : 0.0f;
        bl[t] = t < n ? beta[static_cast<size_t>(r0 + t) * VH + head] : 0.0f;
    }
    __syncthreads();
    if (t < kDeltaChunk) {
        // G_t and G_C, each added in token order.
        float g = 0.0f, gc = 0.0f;
#pragma unroll
        for (int i = 0; i < kDeltaChunk; ++i) {
            gc += dl[i];
            if (i == t) g = gc;
        }
        gl[t] = g;
        eg[t] = expf(g);
        E[t] = eg[t];
        EC[t] = expf(gc - g);
        if (t == 0) GC[0] = expf(gc);
    }
    // K K^T (waves 0, 1) and Q K^T (waves 2, 3): k step s of wave w pairs
    // key slots 64 kh + 32 (w % 2) + s of the lane halves.
    f32x16 acc;
    {
        const int half = wave & 1;
        const float* arow = (wave < 2 ? kl : ql) + li * kDeltaPitch + 64 * kh + 32 * half;
        const float* brow = kl + li * kDeltaPitch + 64 * kh + 32 * half;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int st = 0; st < 32; st += 4) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(arow + st);
            const f32x4 b = *reinterpret_cast<const f32x4*>(brow + st);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, acc, 0, 0, 0);
        }
    }
    __syncthreads();  // every wave is done with ql: it holds the halves now
    float* const part = ql;  // [wave][16][64]
#pragma unroll
    for (int r = 0; r < 16; ++r) part[(wave * 16 + r) * kWave + lane] = acc[r];
    __syncthreads();
    // Entry (i, j) of register r: i = mfma32_row(r, kh), j = li.  Wave 0
    // forms A (held in registers until ql is free again), wave 1 P.
    float dots[16];
    if (wave < 2) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            dots[r] = part[(2 * wave * 16 + r) * kWave + lane] + part[((2 * wave + 1) * 16 + r) * kWave + lane];
    }
    __syncthreads();
    float* const al = ql;  // [32][33]
    if (wave < 2) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = mfma32_row(r, kh), j = li;
            const float d = j <= i ? expf(gl[i] - gl[j]) : 0.0f;
            if (wave == 0) al[i * (kDeltaChunk + 1) + j] = j < i ? bl[i] * d * dots[r] : 0.0f;
            else P[i * kDeltaChunk + j] = d * dots[r];
        }
    }
    __syncthreads();
    // Forward substitution, one thread per column: columns 0..127 of W
    // (right side beta_t e^G_t k_t), 128..255 of U0 (beta_t v_t).
    {
        const bool wcol = t < 128;
        const int c = t & 127;
        const float* src = wcol ? kl : vl;
        float x[kDeltaChunk];
#pragma unroll
        for (int i = 0; i < kDeltaChunk; ++i) {
            float v = (wcol ? bl[i] * eg[i] : bl[i]) * src[i * kDeltaPitch + c];
#pragma unroll
            for (int j = 0; j < i; ++j) v = fmaf(-al[i * (kDeltaChunk + 1) + j], x[j], v);
            x[i] = v;
            // x_i is final before row i + 1's reads of A are issued, so one
            // row of A is live at a time (not all 496 entries).
            asm volatile("" : "+v"(x[i])::"memory");
        }
        float* dst = (wcol ? W : U0) + c;
#pragma unroll
        for (int i = 0; i < kDeltaChunk; ++i) dst[i * 128] = x[i];
    }
}

// The chunks of one value head, in order: a workgroup per (value head,
// 32 value columns), wave a holding the 32 x 32 block of keys 32 a .. of
// the memory in the 32x32 MFMA accumulator layout (lane l: column l % 32,
// keys 8 (r / 4) + 4 (l / 32) + r % 4 in register r).  That layout is also
// the B operand of a k step pairing keys (8 (r / 4) + r % 4, + 4).  Per
// chunk every wave forms its part of W S0 (wave 0 starting from -U0) and
// of Q S0 with the memory as it stands; the W parts are added in LDS in
// wave order to U = U0 - W S0 (the updates, in the accumulator layout: the
// B operand of the next products), every wave adds a quarter of P U (its
// four k steps) to e^G (Q_a S0), and writes that part of O to LDS, added in
// wave order after the next chunk's barrier (each wave stores a quarter of
// the rows); each wave then
// updates its block S = e^G_C S + K^T (e^(G_C - G) U).  The next chunk's
// operands are loaded while the current chunk's run.  Blocks 8 apart run
// on one XCD: the slices of a head are placed so, and share its operands
// in that XCD's L2.
constexpr int kDeltaScanWaves = 4;

__global__ __launch_bounds__(kDeltaScanWaves * kWave) void delta_chunk_scan_kernel(
    const float* __restrict__ qkv, const float* __restrict__ ws, float* __restrict__ memory,
    float* __restrict__ out, int KH, int VH, int KD, int VD, int count) {
    __shared__ __attribute__((aligned(16))) float red[2][2][kDeltaScanWaves][16][kWave];  // [parity][X|O][wave]
    const int slices = VD / 32;
    int blk = blockIdx.x;
    if (VH % 8 == 0) {
        const int x = blk % 8, j = blk / 8;
        blk = ((j / slices) * 8 + x) * slices + j % slices;
    }
    const int head = blk / slices, slice = blk % slices;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int lane = threadIdx.x & (kWave - 1), li = lane & 31, kh = lane >> 5;
    const bool active = wave < KD / 32;
    const int DQK = KH * KD, DQKV = 2 * DQK + VH * VD, DO = VH * VD;
    const int khead = head / (VH / KH);
    const int col = slice * 32 + li;            // this lane's value column
    const int key0 = 32 * (active ? wave : 0);  // first key of the wave's block
    const float* const qrow = qkv + khead * KD + key0;
    const float* const krow = qkv + DQK + khead * KD + key0 + li;
    auto key_of = [&](int r) { return mfma32_row(r, kh); };
    // The memory block: column `col`, keys key0 + key_of(r), four at a time.
    float* const mcol = memory + (static_cast<size_t>(head) * VD + col) * KD + key0;
    f32x16 S;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const f32x4 v = active ? *reinterpret_cast<const f32x4*>(mcol + 8 * q + 4 * kh) : f32x4{0, 0, 0, 0};
        S[4 * q + 0] = v.x; S[4 * q + 1] = v.y; S[4 * q + 2] = v.z; S[4 * q + 3] = v.w;
    }
    // One chunk's operands in this lane's layouts.  Rows past the last
    // token read the last token's q and k: their rows of P, W and U0 are
    // zero, so those values meet only zeros.
    struct Ops {
        f32x16 w, q, k, u0, ec;
        f32x4 p;
        float el, gc;  // e^G of token li, e^G_C
    };
    auto load_ops = [&](int chunk, Ops& o) {
        const float* W = ws + (static_cast<size_t>(chunk) * VH + head) * kDeltaChunkFloats;
        const float* U0 = W + kDeltaTile;
        const float* P = W + 2 * kDeltaTile;
        const float* E = P + kDeltaChunk * kDeltaChunk;
        const float* EC = E + kDeltaChunk;
        const int r0 = chunk * kDeltaChunk;
        const float* q = qrow + static_cast<size_t>(min(r0 + li, count - 1)) * DQKV;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            // A operands of W S0 and Q S0: row li, keys key0 + key_of(4 qd ..).
            const f32x4 w = *reinterpret_cast<const f32x4*>(W + li * 128 + key0 + 8 * qd + 4 * kh);
            const f32x4 qq = *reinterpret_cast<const f32x4*>(q + 8 * qd + 4 * kh);
            // Update scales: tokens key_of(4 qd ..).
            const f32x4 ec = *reinterpret_cast<const f32x4*>(EC + 8 * qd + 4 * kh);
            o.w[4 * qd + 0] = w.x; o.w[4 * qd + 1] = w.y; o.w[4 * qd + 2] = w.z; o.w[4 * qd + 3] = w.w;
            o.q[4 * qd + 0] = qq.x; o.q[4 * qd + 1] = qq.y; o.q[4 * qd + 2] = qq.z; o.q[4 * qd + 3] = qq.w;
            o.ec[4 * qd + 0] = ec.x; o.ec[4 * qd + 1] = ec.y; o.ec[4 * qd + 2] = ec.z; o.ec[4 * qd + 3] = ec.w;
        }
        // A operand of this wave's quarter of P U: row li, tokens key_of(4 wave ..).
        o.p = *reinterpret_cast<const f32x4*>(P + li * kDeltaChunk + 8 * wave + 4 * kh);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            // A operand of K^T U: key key0 + li, token key_of(r).
            o.k[r] = krow[static_cast<size_t>(min(r0 + key_of(r), count - 1)) * DQKV];
        }
        // U0 in the accumulator layout: token key_of(r), column col (every
        // wave loads it, wave 0 uses it: no branch around the loads, whose
        // waits would then cover the prefetch as well).
#pragma unroll
        for (int r = 0; r < 16; ++r) o.u0[r] = U0[key_of(r) * 128 + col];
        o.el = E[li];
        o.gc = EC[kDeltaChunk];
    };
    // Rows key_of(4 wave ..) of O of chunk `chunk`, from its parts in
    // red[parity][1] added in wave order (each wave stores a quarter).  The
    // stores go through a buffer resource that ends at the last row, so rows
    // past it are dropped without a branch.
    auto store_o = [&](int chunk, int parity) {
        const int r0 = chunk * kDeltaChunk;
        const __amdgpu_buffer_rsrc_t rows = __builtin_amdgcn_make_buffer_rsrc(
            out + static_cast<size_t>(r0) * DO, 0, min(kDeltaChunk, count - r0) * DO * 4, kBufferFlags);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float y = red[parity][1][0][4 * wave + e][lane];
#pragma unroll
            for (int a = 1; a < kDeltaScanWaves; ++a) y += red[parity][1][a][4 * wave + e][lane];
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), rows,
                                                  4 * (key_of(4 * wave + e) * DO + head * VD + col), 0, 0);
        }
    };
    const int chunks = (count + kDeltaChunk - 1) / kDeltaChunk;
    auto step = [&](int ch, const Ops& cur, Ops& nxt) {
        load_ops(min(ch + 1, chunks - 1), nxt);  // unconditional: see U0 above
        const int par = ch & 1;
        f32x16 X, Y;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            X[r] = wave == 0 ? -cur.u0[r] : 0.0f;
            Y[r] = 0.0f;
        }
        // e^G (Q S0) with e^G_li on the A operand's row li.
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            X = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.w[r], S[r], X, 0, 0, 0);
            Y = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.q[r] * cur.el, S[r], Y, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) red[par][0][wave][r][lane] = X[r];
        __syncthreads();
        if (ch > 0) store_o(ch - 1, par ^ 1);
        // U = U0 - W S0: minus the parts, added in wave order.
        f32x16 U;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float x = red[par][0][0][r][lane];
#pragma unroll
            for (int a = 1; a < kDeltaScanWaves; ++a) x += red[par][0][a][r][lane];
            U[r] = -x;
        }
        // This wave's part of O: e^G (Q_a S0) + P[:, tokens key_of(4 wave ..)] U.
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if ((r >> 2) == wave) Y = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.p[r & 3], U[r], Y, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) red[par][1][wave][r][lane] = Y[r];
        if (active) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                S[r] *= cur.gc;
                U[r] *= cur.ec[r];
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) S = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.k[r], U[r], S, 0, 0, 0);
        }
    };
    Ops a, b;
    load_ops(0, a);
    for (int ch = 0; ch < chunks; ch += 2) {
        step(ch, a, b);
        if (ch + 1 < chunks) step(ch + 1, b, a);
    }
    __syncthreads();
    store_o(chunks - 1, (chunks - 1) & 1);
    if (active) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<f32x4*>(mcol + 8 * q + 4 * kh) = f32x4{S[4 * q + 0], S[4 * q + 1], S[4 * q + 2], S[4 * q + 3]};
    }
}

// One decode token of the gated delta rule (engine.cpp:262-316) in the
// layout of delta_scan_kernel: a value head's columns over kScanSlices
// workgroups of 4 waves, lane l of wave w owning column 32 slice + 8 w + l / 8
// and keys 16 (l % 8) .. + 15, the sums over keys DPP adds inside row halves,
// and the scan's arithmetic per token (k S once scaled by e^decay, S e^decay +
// k (beta delta), q S).  The token's causal conv runs here too (conv_fetch, conv_apply):
// thread t convolves q channel t (t < 128) or k channel t - 128 of the key
// head and the first kScanCols threads the slice's v channels, from history
// copy p % 2 into copy (p + 1) % 2 -- q and k only from slice 0 of the key
// head's first value head; then the L2 norms of q and k (q also divided by
// sqrt(KD)), beta = sigmoid(b) and e^decay as delta_prep_kernel forms them.
// Writes q S unnormalised and, for the gated RMSNorm that follows in the out
// projection's input staging (GatedNormInput), gate = norm * silu(z) of each
// column, formed once here (delta_norm_kernel, the fallback, uses z itself).
__global__ __launch_bounds__(kScanThreads) void delta_step_kernel(
    const float* __restrict__ qkv, const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ z, const float* __restrict__ alog, const uint16_t* __restrict__ dt,
    const float* __restrict__ norm, float* __restrict__ memory, float* __restrict__ out,
    float* __restrict__ gate, const uint16_t* __restrict__ conv_w, float* __restrict__ history,
    const int* __restrict__ position, int CK, int KH, int VH, int KD, int VD) {
    __shared__ __attribute__((aligned(16))) float qk[256];  // q (0 .. 127), k (128 .. 255), zeros past KD
    __shared__ float vs[kScanCols];
    __shared__ float squares[kScanThreads / kWave];
    const int head = blockIdx.x / kScanSlices, slice = blockIdx.x % kScanSlices;
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1), wave = t / kWave;
    const int DQK = KH * KD, DO = VH * VD, DQKV = 2 * DQK + DO;
    const int per = VH / KH, kh = head / per;
    const int cl = wave * (kWave / kScanGroups) + lane / kScanGroups;  // column within the slice
    const int c = slice * kScanCols + cl, k0 = (lane % kScanGroups) * kScanKeys;
    const bool col = c < VD;
    float* S = memory + (static_cast<size_t>(head) * VD + (col ? c : 0)) * KD;  // column c
    // Every input is requested before any is used -- the memory columns,
    // the head's gate parameters, the conv inputs with both history copies
    // (the position only picks one), the output gate's norm and z -- so the
    // step waits for one round trip to memory instead of four.
    float s[kScanKeys];
    load_keys<kScanKeys>(S, k0, KD, col, s);
    const int pos = *position;
    const float a_in = a[head], b_in = b[head];
    const float alog_h = alog[head];
    const uint16_t dt_h = dt[head];
    const bool writer = lane % kScanGroups == 0 && col;
    const size_t at = static_cast<size_t>(head) * VD + c;
    const float norm_c = writer ? norm[c] : 0.0f;
    const float z_at = writer ? z[at] : 0.0f;
    const size_t copy = static_cast<size_t>(DQKV) * (CK - 1);
    const bool qk_writer = head % per == 0 && slice == 0;
    // q | k channel of this thread (t < 128: q, else k).
    const int ch = t & 127;
    const int ci_qk = (t < 128 ? 0 : DQK) + kh * KD + ch;
    ConvInputs in_qk{}, in_v{};
    if (ch < KD) conv_fetch(in_qk, qkv[ci_qk], history, copy, conv_w, ci_qk, CK);
    const int cv = slice * kScanCols + t;
    const int ci_v = 2 * DQK + head * VD + cv;  // each v channel belongs to one slice
    const bool has_v = t < kScanCols && cv < VD;
    if (has_v) conv_fetch(in_v, qkv[ci_v], history, copy, conv_w, ci_v, CK);
    const int parity = pos & 1;
    float* hout = history + static_cast<size_t>(parity ^ 1) * copy;
    float x = 0.0f;
    if (ch < KD)
        x = conv_apply(in_qk, parity, CK, qk_writer ? hout + static_cast<size_t>(ci_qk) * (CK - 1) : nullptr);
    if (t < kScanCols) vs[t] = has_v ? conv_apply(in_v, parity, CK, hout + static_cast<size_t>(ci_v) * (CK - 1)) : 0.0f;
    // L2 norms: waves 0, 1 hold q, waves 2, 3 hold k.
    const float sq = wave_sum_f32(x * x);
    if (lane == 0) squares[wave] = sq;
    __syncthreads();
    if (t < 128) qk[t] = x * (1.0f / sqrtf(squares[0] + squares[1] + kEps)) / sqrtf(static_cast<float>(KD));
    else qk[t] = x * (1.0f / sqrtf(squares[2] + squares[3] + kEps));
    __syncthreads();
    const float bb = sigmoid_ref(b_in);
    const float sc = expf(-expf(alog_h) * softplus_ref(a_in + bf16_value(dt_h)));
    const f32x4* kp = reinterpret_cast<const f32x4*>(qk + 128 + k0);
    const f32x4* qp = reinterpret_cast<const f32x4*>(qk + k0);
    float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
    for (int j4 = 0; j4 < kScanKeys / 4; ++j4) {
        const f32x4 kk = kp[j4];
        p0 = fmaf(kk.x, s[4 * j4 + 0], p0);
        p1 = fmaf(kk.y, s[4 * j4 + 1], p1);
        p0 = fmaf(kk.z, s[4 * j4 + 2], p0);
        p1 = fmaf(kk.w, s[4 * j4 + 3], p1);
    }
    float pred = p0 + p1;
    pred += dpp_f32<0xB1>(pred);   // the eight key groups: pairs,
    pred += dpp_f32<0x4E>(pred);   // quads,
    pred += dpp_f32<0x141>(pred);  // the two quads of the row half
    const float bd = bb * (vs[cl] - sc * pred);  // beta (v - k S e^decay)
    float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int j4 = 0; j4 < kScanKeys / 4; ++j4) {
        const f32x4 kk = kp[j4], qq = qp[j4];
        s[4 * j4 + 0] = fmaf(s[4 * j4 + 0], sc, kk.x * bd);
        s[4 * j4 + 1] = fmaf(s[4 * j4 + 1], sc, kk.y * bd);
        s[4 * j4 + 2] = fmaf(s[4 * j4 + 2], sc, kk.z * bd);
        s[4 * j4 + 3] = fmaf(s[4 * j4 + 3], sc, kk.w * bd);
        o0 = fmaf(qq.x, s[4 * j4 + 0], o0);
        o1 = fmaf(qq.y, s[4 * j4 + 1], o1);
        o0 = fmaf(qq.z, s[4 * j4 + 2], o0);
        o1 = fmaf(qq.w, s[4 * j4 + 3], o1);
    }
    float o = o0 + o1;
    o += dpp_f32<0xB1>(o);
    o += dpp_f32<0x4E>(o);
    o += dpp_f32<0x141>(o);
    if (writer) {
        out[at] = o;
        gate[at] = norm_c * silu_ref(z_at);
    }
    store_keys<kScanKeys>(S, k0, KD, col, s);
}

__global__ __launch_bounds__(128) void delta_norm_kernel(float* __restrict__ out, const float* __restrict__ z,
                                                         const float* __restrict__ norm, int VH, int VD) {
    __shared__ float partial[128 / kWave];
    const int head = blockIdx.x, r = blockIdx.y;
    const int t = threadIdx.x;
    const size_t at = static_cast<size_t>(r) * VH * VD + head * VD + t;
    const float x = t < VD ? out[at] : 0.0f;
    const float sq = block_sum<128>(x * x, partial);
    if (t < VD) {
        const float g = 1.0f / sqrtf(sq / static_cast<float>(VD) + kEps);
        out[at] = x * (g * norm[t] * silu_ref(z[at]));
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

// Row r = blockIdx.y at position *position + r.  Query heads (blockIdx.x <
// AH): split the q|gate rows, norm and rotate q; key/value heads: norm and
// rotate k and append k and v to the cache (engine.cpp:318-343).  AD <= 256.
__global__ __launch_bounds__(kHeadThreads) void attention_prep_kernel(
    const float* __restrict__ query_and_gate, const float* __restrict__ key, const float* __restrict__ value,
    const uint16_t* __restrict__ qnorm, const uint16_t* __restrict__ knorm, const int* __restrict__ position,
    float* __restrict__ query, float* __restrict__ gate, float* __restrict__ key_cache,
    float* __restrict__ value_cache, int AH, int KVH, int AD, int RD) {
    __shared__ float x[256], partial[kHeadThreads / kWave];
    const int t = threadIdx.x;
    const int r = blockIdx.y;
    const int pos = *position + r;
    const int AS = AH * AD, KVW = KVH * AD;
    if (blockIdx.x < AH) {
        const int head = blockIdx.x;
        const float* qg = query_and_gate + static_cast<size_t>(r) * 2 * AS;
        if (t < AD) {
            x[t] = qg[head * 2 * AD + t];
            gate[static_cast<size_t>(r) * AS + head * AD + t] = qg[head * 2 * AD + AD + t];
        }
        __syncthreads();
        norm_rope(x, qnorm, AD, RD, pos, partial);
        if (t < AD) query[static_cast<size_t>(r) * AS + head * AD + t] = x[t];
    } else {
        const int head = blockIdx.x - AH;
        if (t < AD) x[t] = key[static_cast<size_t>(r) * KVW + head * AD + t];
        __syncthreads();
        norm_rope(x, knorm, AD, RD, pos, partial);
        const size_t at = (static_cast<size_t>(pos) * KVH + head) * AD;
        if (t < AD) {
            key_cache[at + t] = x[t];
            value_cache[at + t] = value[static_cast<size_t>(r) * KVW + head * AD + t];
        }
    }
}

// Sum over the 64 lanes of each of 64 values: afterwards lane L holds the
// total of value L.  Six exchange levels, one per lane-index bit from the top:
// at each, a lane keeps the half of its values that its bit selects (the upper
// half when the bit is set) and adds its partner's copy of that half, so the
// levels move 32 + 16 + 8 + 4 + 2 + 1 values instead of 64 full reductions.
// Bits 5 and 4 pair lanes L and L ^ 32 / L ^ 16 by the gfx950 lane swaps
// (v_permlane32_swap, v_permlane16_swap); bits 3 .. 0 by DPP (row_mirror,
// row_half_mirror, then the two quad permutations), whose partners differ
// from the lane in the level's bit and agree in every bit above it.
__device__ __forceinline__ float transpose_sum64(float (&v)[64]) {
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 32]), false, false);
        v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 16]), false, false);
        v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const int lane = threadIdx.x & (kWave - 1);
    auto level = [&](auto ctrl, int half, bool upper) {
#pragma unroll
        for (int k = 0; k < half; ++k) {
            const float keep = upper ? v[k + half] : v[k];
            const float send = upper ? v[k] : v[k + half];
            v[k] = keep + dpp_f32<decltype(ctrl)::value>(send);
        }
    };
    level(std::integral_constant<int, 0x140>{}, 8, (lane & 8) != 0);
    level(std::integral_constant<int, 0x141>{}, 4, (lane & 4) != 0);
    level(std::integral_constant<int, 0x4E>{}, 2, (lane & 2) != 0);
    level(std::integral_constant<int, 0xB1>{}, 1, (lane & 1) != 0);
    return v[0];
}

// Decode attention of the query row at *position for the G = AH / KVH query
// heads that share KV head blockIdx.x / splits (engine.cpp:344-361: scores
// q . k / sqrt(AD), softmax, sum of weights times v), over position range
// blockIdx.x % splits of 0 .. *position.  A range is taken in blocks of
// B = 4 * 64 / GP positions (GP = G rounded up to 4 or 8): wave w holds the K
// and V rows of positions w, w + 4, ... of a block, lane l elements 4l .. 4l +
// 3 of each, every load of a block requested at once and each row loaded once
// for all G heads.  The lane products q_g . k_u of a wave's 64 (row, head)
// pairs reduce together in transpose_sum64; the scores go to LDS, where wave
// w runs the online softmax of heads w, w + 4 with wave reductions (a running
// maximum rescales the running sum and accumulators), so no score buffer
// bounds the context.  Each wave accumulates weight times v over its own rows
// (four outputs per lane per head); the four waves' accumulators add in wave
// order at the end.  Each head's range maximum, sum and accumulator go to
// `partial` for attention_combine_kernel (empty ranges leave m = -inf, l = 0).
// AD <= 256 and a multiple of 4, G <= kMaxGroup.
constexpr int kAttnSplits = 128;  // ranges per KV head for a decode step
constexpr int kMaxGroup = 8;
constexpr int kChunk = 4096;     // default rows of a prefill chunk
constexpr size_t kGemmScratchMax = static_cast<size_t>(512) << 20;  // K-split partial sums, at most

template <int GP>
__global__ __launch_bounds__(kHeadThreads) void attention_kernel(
    const float* __restrict__ query, const float* __restrict__ key_cache, const float* __restrict__ value_cache,
    const int* __restrict__ position, float* __restrict__ partial, int AH, int KVH, int AD, int splits) {
    constexpr int kWaves = kHeadThreads / kWave;
    static_assert(GP == 4 || GP == 8, "64 (row, head) pairs per wave");
    constexpr int R = kWave / GP;  // rows per wave per block
    constexpr int B = kWaves * R;  // positions per block
    // Scores, then weights, wave-major: sc[g][w * R + u] is position u * 4 + w.
    __shared__ __attribute__((aligned(16))) float sc[GP][B];
    __shared__ float head_m[GP], head_l[GP], head_alpha[GP];
    __shared__ __attribute__((aligned(16))) float red[kWaves - 1][GP][256];
    const int kv = blockIdx.x / splits, split = blockIdx.x % splits;
    const int G = AH / KVH;
    const int n = *position + 1;
    const int per = (n + splits - 1) / splits;
    const int t0 = min(n, split * per), t1 = min(n, t0 + per);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const size_t KVW = static_cast<size_t>(KVH) * AD;
    const float* kbase = key_cache + static_cast<size_t>(kv) * AD + 4 * lane;
    const float* vbase = value_cache + static_cast<size_t>(kv) * AD + 4 * lane;
    const float divisor = sqrtf(static_cast<float>(AD));
    const bool kl = 4 * lane < AD;
    f32x4 kr[R], vr[R];
    auto load_block = [&](int b0) {
        const int nb = min(B, t1 - b0);
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const int j = u * kWaves + wave;
            kr[u] = j < nb && kl ? *reinterpret_cast<const f32x4*>(kbase + static_cast<size_t>(b0 + j) * KVW) : f32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const int j = u * kWaves + wave;
            vr[u] = j < nb && kl ? *reinterpret_cast<const f32x4*>(vbase + static_cast<size_t>(b0 + j) * KVW) : f32x4{0, 0, 0, 0};
        }
    };
    if (t0 < t1) load_block(t0);
    f32x4 q[GP];
#pragma unroll
    for (int g = 0; g < GP; ++g)
        q[g] = g < G && kl ? *reinterpret_cast<const f32x4*>(query + (kv * G + g) * AD + 4 * lane) : f32x4{0, 0, 0, 0};
    f32x4 acc[GP];
#pragma unroll
    for (int g = 0; g < GP; ++g) acc[g] = f32x4{0, 0, 0, 0};
    if (threadIdx.x < GP) {
        head_m[threadIdx.x] = -INFINITY;
        head_l[threadIdx.x] = 0.0f;
    }
    __syncthreads();
    // After transpose_sum64, lane L holds the score of row u = L / GP, head g = L % GP.
    const int my_u = lane / GP, my_g = lane % GP;
    for (int b0 = t0; b0 < t1; b0 += B) {
        const int nb = min(B, t1 - b0);
        if (b0 != t0) load_block(b0);
        float v[64];
#pragma unroll
        for (int u = 0; u < R; ++u) {
#pragma unroll
            for (int g = 0; g < GP; ++g) {
                float x = q[g].x * kr[u].x;
                x = fmaf(q[g].y, kr[u].y, x);
                x = fmaf(q[g].z, kr[u].z, x);
                x = fmaf(q[g].w, kr[u].w, x);
                v[u * GP + g] = x;
            }
        }
        const float s = transpose_sum64(v);
        sc[my_g][wave * R + my_u] = s / divisor;
        __syncthreads();
        for (int g = wave; g < G; g += kWaves) {
            // lane = w * R + u holds position u * 4 + w.
            const bool valid = lane < B && (lane % R) * kWaves + lane / R < nb;
            const float sj = valid ? sc[g][lane] : -INFINITY;
            const float mo = head_m[g];
            const float mn = fmaxf(mo, wave_max_f32(sj));
            const float pj = valid ? expf(sj - mn) : 0.0f;
            const float ps = wave_sum_f32(pj);
            if (lane < B) sc[g][lane] = pj;
            if (lane == 0) {
                const float alpha = expf(mo - mn);  // 0 for the first block (mo = -inf)
                head_alpha[g] = alpha;
                head_m[g] = mn;
                head_l[g] = head_l[g] * alpha + ps;
            }
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < GP; ++g) {
            if (g < G) {
                const float alpha = head_alpha[g];
                f32x4 a = {acc[g].x * alpha, acc[g].y * alpha, acc[g].z * alpha, acc[g].w * alpha};
#pragma unroll
                for (int u0 = 0; u0 < R; u0 += 4) {
                    const f32x4 p = *reinterpret_cast<const f32x4*>(&sc[g][wave * R + u0]);
                    const float pw[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        a.x = fmaf(pw[d], vr[u0 + d].x, a.x);
                        a.y = fmaf(pw[d], vr[u0 + d].y, a.y);
                        a.z = fmaf(pw[d], vr[u0 + d].z, a.z);
                        a.w = fmaf(pw[d], vr[u0 + d].w, a.w);
                    }
                }
                acc[g] = a;
            }
        }
        __syncthreads();
    }
    // The waves' partial accumulators, summed in wave order.
    if (wave > 0 && kl) {
#pragma unroll
        for (int g = 0; g < GP; ++g)
            if (g < G) *reinterpret_cast<f32x4*>(&red[wave - 1][g][4 * lane]) = acc[g];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int g = 0; g < GP; ++g) {
            if (g >= G) continue;
            float* p = partial + (static_cast<size_t>(kv * G + g) * splits + split) * (AD + 2);
            if (kl) {
                f32x4 a = acc[g];
#pragma unroll
                for (int w = 0; w < kWaves - 1; ++w) {
                    const f32x4 o = *reinterpret_cast<const f32x4*>(&red[w][g][4 * lane]);
                    a.x += o.x; a.y += o.y; a.z += o.z; a.w += o.w;
                }
                p[4 * lane + 0] = a.x; p[4 * lane + 1] = a.y; p[4 * lane + 2] = a.z; p[4 * lane + 3] = a.w;
            }
            if (lane == 0) {
                p[AD] = head_m[g];
                p[AD + 1] = head_l[g];
            }
        }
    }
}

// Prefill attention on the matrix cores, causal over positions 0 ..
// *position + row, FP32 MFMA (v_mfma_f32_32x32x2_f32, exact products, FP32
// sums).  A workgroup takes one tile of 32 query rows (the longest tiles
// first) for up to kFlashWaves query heads of one KV head, one wave per
// head.  Per block of 32 positions the K and V rows go global -> LDS once
// for all of the workgroup's heads, by direct-to-LDS buffer loads into a
// double buffer: the next block's copy is in flight while the current one is
// used, and one barrier per block separates them.  Each wave forms S^T = K
// Q^T (rows positions, columns queries), so lane l holds 16 of query l %
// 32's scores and lane l ^ 32 the other 16: the online-softmax maximum and
// sum of a query are a 16-register reduction and one swap between the
// wave's halves.  In the same registers exp(S^T - m) is the A operand of P V
// (the pair index of the MFMA k step is the half of the wave in both), so P
// is never moved; the per-query rescale factors reach the output rows
// through a 32-float LDS transpose.  Q stays in registers.  LDS rows are
// padded (K pitch 260, V pitch 264 floats) so the K row reads of 16 lanes
// and the V column reads of the two wave halves fall in distinct banks.
// Scores are q . k / sqrt(AD) as engine.cpp:344-361; AD a multiple of 32, at
// most 256.
constexpr int kFlashQ = 32;
constexpr int kFlashWaves = 4;
constexpr int kFlashKPitch = 260, kFlashVPitch = 264;
constexpr size_t kFlashLds =
    (2 * kFlashQ * (kFlashKPitch + kFlashVPitch) + kFlashWaves * kFlashQ) * sizeof(float);

__global__ __launch_bounds__(kFlashWaves * kWave, 1) void attention_prefill_kernel(
    const float* __restrict__ query, const float* __restrict__ gate, const float* __restrict__ key_cache,
    const float* __restrict__ value_cache, const int* __restrict__ position, float* __restrict__ out, int AH,
    int KVH, int AD, int count) {
    extern __shared__ __attribute__((aligned(16))) float flash_lds[];
    float* const kl = flash_lds;                                  // [2][32][kFlashKPitch]
    float* const vl = kl + 2 * kFlashQ * kFlashKPitch;            // [2][32][kFlashVPitch]
    const int G = AH / KVH;
    const int subs = (G + kFlashWaves - 1) / kFlashWaves;
    const int kv = blockIdx.x / subs, sub = blockIdx.x % subs;
    const int q0 = (gridDim.y - 1 - blockIdx.y) * kFlashQ;  // longest tiles first
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x & (kWave - 1), li = lane & 31, kh = lane >> 5;
    float* const row_scale = vl + 2 * kFlashQ * kFlashVPitch + wave * kFlashQ;
    const int hg = sub * kFlashWaves + wave;  // head within the KV head's group
    const bool active = hg < G;
    const int head = kv * G + (active ? hg : 0);
    const int AS = AH * AD, NB = AD / 32;
    const size_t KVW = static_cast<size_t>(KVH) * AD;
    const int p0 = *position;
    const int rows = min(kFlashQ, count - q0);
    const int last = p0 + q0 + rows - 1;  // the tile's last query position
    const int my_pos = p0 + q0 + li;      // this lane's query (S^T column)
    const bool my_valid = li < rows;
    const float divisor = sqrtf(static_cast<float>(AD));

    // Rows of block b0 into buffer `buf`: wave w copies K and V rows 8 w ..
    // 8 w + 7 (positions past `last` repeat row `last`; their scores are
    // masked and their weights are zero).  Each row is one 16-byte-per-lane
    // load of AD floats; lanes past the row read zeros.
    auto copy_block = [&](int b0, int buf) {
#pragma unroll
        for (int r = 0; r < kFlashQ / kFlashWaves; ++r) {
            const int p = wave * (kFlashQ / kFlashWaves) + r;
            const size_t at = static_cast<size_t>(min(b0 + p, last)) * KVW + static_cast<size_t>(kv) * AD;
            const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(key_cache + at), 0, AD * 4, kBufferFlags);
            const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(value_cache + at), 0, AD * 4, kBufferFlags);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                kr, (__attribute__((address_space(3))) void*)(kl + (buf * kFlashQ + p) * kFlashKPitch), 16, 16 * lane,
                0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                vr, (__attribute__((address_space(3))) void*)(vl + (buf * kFlashQ + p) * kFlashVPitch), 16, 16 * lane,
                0, 0, 0);
        }
    };
    copy_block(0, 0);

    // Q row li of this wave's head, dims 32 b + 16 kh + (0 .. 15) of each
    // 32-dim block b.
    f32x4 qf[8][4];
    {
        const float* qr = query + static_cast<size_t>(q0 + min(li, rows - 1)) * AS + head * AD;
#pragma unroll
        for (int b = 0; b < 8; ++b)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                qf[b][j] = b < NB ? *reinterpret_cast<const f32x4*>(qr + 32 * b + 16 * kh + 4 * j) : f32x4{0, 0, 0, 0};
    }
    f32x16 o[8];
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;
    float m = -INFINITY, l = 0.0f;  // of query li (the same in lanes li and li + 32)
    int buf = 0;
    for (int b0 = 0; b0 <= last; b0 += 32, buf ^= 1) {
        // This block's rows have landed (every wave's copies), and every wave
        // is done with the other buffer: the next block may overwrite it.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (b0 + 32 <= last) copy_block(b0 + 32, buf ^ 1);
        if (!active) continue;
        const float* kb = kl + buf * kFlashQ * kFlashKPitch;
        const float* vb = vl + buf * kFlashQ * kFlashVPitch;
        // S^T[p][q] for positions b0 + p: two accumulators over alternate
        // 32-dim blocks, so consecutive MFMAs do not wait on each other.
        f32x16 s0, s1;
#pragma unroll
        for (int r = 0; r < 16; ++r) s0[r] = s1[r] = 0.0f;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            if (b < NB) {
                f32x4 kf[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    kf[j] = *reinterpret_cast<const f32x4*>(kb + li * kFlashKPitch + 32 * b + 16 * kh + 4 * j);
#pragma unroll
                for (int st = 0; st < 16; ++st) {
                    if (b & 1)
                        s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[st >> 2][st & 3], qf[b][st >> 2][st & 3], s1, 0, 0, 0);
                    else
                        s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[st >> 2][st & 3], qf[b][st >> 2][st & 3], s0, 0, 0, 0);
                }
            }
        }
        // Scores, causal mask, block maximum of query li.
        float sc[16];
        float bm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int p = b0 + 8 * (r >> 2) + 4 * kh + (r & 3);
            const float v = (s0[r] + s1[r]) / divisor;
            sc[r] = p <= my_pos && p <= last ? v : -INFINITY;
            bm = fmaxf(bm, sc[r]);
        }
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        const float mn = my_valid ? fmaxf(m, bm) : 0.0f;
        float ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            sc[r] = my_valid ? expf(sc[r] - mn) : 0.0f;  // masked: exp(-inf) = 0
            ps += sc[r];
        }
        ps += __shfl_xor(ps, 32);
        const float alpha = my_valid ? expf(m - mn) : 0.0f;  // 0 on the first block
        l = l * alpha + ps;
        m = mn;
        // Rescale the output rows: row q of register r is query
        // 8 (r / 4) + 4 kh + r % 4; its factor comes from lane q.
        if (kh == 0) row_scale[li] = alpha;
        wave_lds_sync();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float a = row_scale[8 * (r >> 2) + 4 * kh + (r & 3)];
#pragma unroll
            for (int t = 0; t < 8; ++t) o[t][r] *= a;
        }
        wave_lds_sync();
        // O += P V: k step u pairs position 8 (u / 4) + 4 kh + u % 4 with
        // register u of P, lane column li with output dim 32 t + li.
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            if (t < NB) {
                float vv[16];
#pragma unroll
                for (int u = 0; u < 16; ++u)
                    vv[u] = vb[(8 * (u >> 2) + 4 * kh + (u & 3)) * kFlashVPitch + 32 * t + li];
#pragma unroll
                for (int u = 0; u < 16; ++u) o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(sc[u], vv[u], o[t], 0, 0, 0);
            }
        }
    }
    if (!active) return;
    // out = O / l * sigmoid(gate) for the tile's valid rows.
    if (kh == 0) row_scale[li] = my_valid ? 1.0f / l : 0.0f;
    wave_lds_sync();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int q = 8 * (r >> 2) + 4 * kh + (r & 3);
        if (q < rows) {
            const float inv = row_scale[q];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                if (t < NB) {
                    const size_t at = static_cast<size_t>(q0 + q) * AS + head * AD + 32 * t + li;
                    out[at] = o[t][r] * inv * sigmoid_ref(gate[at]);
                }
            }
        }
    }
}

// out = (sum_s exp(m_s - M) acc_s) / (sum_s exp(m_s - M) l_s) * sigmoid(gate)
// over the kAttnSplits ranges s of head blockIdx.x of row r = blockIdx.z, M
// their largest maximum (empty ranges have m = -inf and weight 0).  A
// workgroup takes kCombCols output elements (blockIdx.y): thread t sums
// ranges (t / kCombCols) * kPer .. + kPer of element t % kCombCols, every load
// requested at once, and the groups' sums add in group order.
constexpr int kCombCols = 32;
__global__ __launch_bounds__(kHeadThreads) void attention_combine_kernel(const float* __restrict__ partial,
                                                           const float* __restrict__ gate,
                                                           float* __restrict__ out, int AH, int AD) {
    constexpr int kGroups = kHeadThreads / kCombCols;
    constexpr int kPer = kAttnSplits / kGroups;
    static_assert(kAttnSplits % kGroups == 0 && kAttnSplits <= kHeadThreads, "whole groups of ranges");
    __shared__ float w[kAttnSplits], red[kHeadThreads / kWave];
    __shared__ float part[kGroups][kCombCols];
    __shared__ float total;
    const int head = blockIdx.x, r = blockIdx.z;
    const float* p = partial + (static_cast<size_t>(r) * AH + head) * kAttnSplits * (AD + 2);
    const int t = threadIdx.x;
    const int e = blockIdx.y * kCombCols + t % kCombCols, grp = t / kCombCols;
    float v[kPer];
#pragma unroll
    for (int s = 0; s < kPer; ++s) v[s] = e < AD ? p[(grp * kPer + s) * (AD + 2) + e] : 0.0f;
    const float m = t < kAttnSplits ? p[t * (AD + 2) + AD] : -INFINITY;
    const float M = block_max<kHeadThreads>(m, red);
    const float ws = t < kAttnSplits && m != -INFINITY ? expf(m - M) : 0.0f;
    if (t < kAttnSplits) w[t] = ws;
    const float L = block_sum<kHeadThreads>(t < kAttnSplits ? ws * p[t * (AD + 2) + AD + 1] : 0.0f, red);
    if (t == 0) total = L;
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < kPer; ++s) acc = fmaf(w[grp * kPer + s], v[s], acc);
    part[grp][t % kCombCols] = acc;
    __syncthreads();
    if (t < kCombCols && e < AD) {
        float a = part[0][t];
#pragma unroll
        for (int g2 = 1; g2 < kGroups; ++g2) a += part[g2][t];
        const size_t at = static_cast<size_t>(r) * AH * AD + head * AD + e;
        out[at] = a / total * sigmoid_ref(gate[at]);
    }
}
// h = silu(gate) * up (engine.cpp:371-376), in place in gate.
__global__ __launch_bounds__(256) void swiglu_kernel(float* __restrict__ gate, const float* __restrict__ up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) gate[i] = silu_ref(gate[i]) * up[i];
}

// gate = gate * up in place, for a gate that already holds silu(gate): the
// second half of swiglu_kernel's arithmetic.
__global__ __launch_bounds__(256) void product_kernel(float* __restrict__ gate, const float* __restrict__ up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) gate[i] = gate[i] * up[i];
}

// Element i of x in the matvec kernels' padded LDS copy.
__device__ __forceinline__ float* lds_x(uint8_t* xl, int i) {
    return reinterpret_cast<float*>(xl + x_block_offset(i / kBlock) + 4 * (i % kBlock));
}

// Input staging for a decode step's down projection: x = silu(gate) * up
// (engine.cpp:371-376; swiglu_kernel's arithmetic), where the gate|up
// matvec has already stored silu(gate) (MultiRows::silu_mask, once per row),
// so each workgroup forms x with one multiply per value on the way into LDS
// -- the same two roundings as swiglu_kernel, bit for bit.  (Evaluating silu
// here instead, in every one of the launch's workgroups, cost ~5 us per
// launch at the 27B shape.)
struct SwiGLUInput {
    const float* up;
    __device__ void stage(const float* silu_gate, uint8_t* xl, int bpr, float* /*work*/) const {
        const f32x4* g = reinterpret_cast<const f32x4*>(silu_gate);
        const f32x4* u = reinterpret_cast<const f32x4*>(up);
        for (int c = threadIdx.x; c < bpr * 8; c += blockDim.x) {
            const f32x4 a = g[c], b = u[c];
            *reinterpret_cast<f32x4*>(xl + x_block_offset(c >> 3) + 16 * (c & 7)) =
                f32x4{a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w};
        }
        __syncthreads();
    }
};

// Input staging of a DeltaNet layer's out projection in a decode step
// (mv_pipe_kernel's `In`): x = the gated RMSNorm of the delta rule's raw
// output o (engine.cpp:234-239): per value head h, g = 1 / sqrt(mean(o_h^2) +
// eps), x = o * (g * gate), gate = norm[j] * silu(z) formed by
// delta_step_kernel.  Every workgroup forms it on the way into LDS: each
// thread loads its chunks of o and gate in one round trip (the first kHeld
// stay in registers).  With 128-value heads and every chunk held, a head's
// sum of squares is the 32-lane DPP sum of its 32 chunks' threads (each
// adding its own four squares with FMAs in order), and each thread scales and
// stores its chunks at once.  Otherwise o is copied to LDS, 16-lane groups
// take the heads (group G: heads G, G + groups, ...), lane i summing the
// squares of columns i, i + 16, ... in order with FMAs and the group adding
// its lanes with DPP, then each thread scales its chunks.  Either way every
// workgroup holds the same scales.  Requires VD % 4 == 0 and at most 256
// heads (the scales use the 1 KB work area).
struct GatedNormInput {
    static constexpr int kHeld = 6;
    const float* gate;  // [VH * VD]: norm[j] * silu(z)
    int VD;
    __device__ void stage(const float* o, uint8_t* xl, int bpr, float* work) const {
        const int chunks = bpr * 8;
        const int heads = bpr * kBlock / VD;
        const int B = blockDim.x;
        const f32x4* os = reinterpret_cast<const f32x4*>(o);
        const f32x4* gs = reinterpret_cast<const f32x4*>(gate);
        auto at = [&](int ck) { return reinterpret_cast<f32x4*>(xl + x_block_offset(ck >> 3) + 16 * (ck & 7)); };
        f32x4 orr[kHeld], grr[kHeld];
#pragma unroll
        for (int k = 0; k < kHeld; ++k) {
            const int ck = threadIdx.x + k * B;
            if (ck < chunks) {
                orr[k] = os[ck];
                grr[k] = gs[ck];
            }
        }
        if (VD == 128 && chunks <= kHeld * B) {
            // Every chunk is held, and the 32 chunks of a 128-value head are
            // the k-th chunks of 32 consecutive threads (B is a multiple of
            // 64): each head's sum of squares is a 32-lane DPP sum of the
            // threads' own four squares, with no LDS round trip.
#pragma unroll
            for (int k = 0; k < kHeld; ++k) {
                const int ck = threadIdx.x + k * B;
                const bool mine = ck < chunks;
                float sq = 0.0f;
                if (mine) {
                    sq = fmaf(orr[k].x, orr[k].x, sq);
                    sq = fmaf(orr[k].y, orr[k].y, sq);
                    sq = fmaf(orr[k].z, orr[k].z, sq);
                    sq = fmaf(orr[k].w, orr[k].w, sq);
                }
                const float total = group_sum<32>(sq);
                if (mine) {
                    const float g = 1.0f / sqrtf(total / static_cast<float>(VD) + kEps);
                    f32x4 v = orr[k];
                    v.x = v.x * (g * grr[k].x);
                    v.y = v.y * (g * grr[k].y);
                    v.z = v.z * (g * grr[k].z);
                    v.w = v.w * (g * grr[k].w);
                    *at(ck) = v;
                }
            }
            __syncthreads();
            return;
        }
#pragma unroll
        for (int k = 0; k < kHeld; ++k) {
            const int ck = threadIdx.x + k * B;
            if (ck < chunks) *at(ck) = orr[k];
        }
        for (int ck = threadIdx.x + kHeld * B; ck < chunks; ck += B) *at(ck) = os[ck];
        __syncthreads();
        const int li = threadIdx.x & 15, group = threadIdx.x / 16, groups = B / 16;
        for (int h0 = 0; h0 < heads; h0 += groups) {
            // Every lane of the block takes part (group_sum needs whole waves).
            const int h = h0 + group;
            float sq = 0.0f;
            if (h < heads)
                for (int j = li; j < VD; j += 16) {
                    const float v = *lds_x(xl, h * VD + j);
                    sq = fmaf(v, v, sq);
                }
            const float total = group_sum<16>(sq);
            if (li == 0 && h < heads) work[h] = 1.0f / sqrtf(total / static_cast<float>(VD) + kEps);
        }
        __syncthreads();
        auto put = [&](int ck, f32x4 v, f32x4 w) {
            const float g = work[4 * ck / VD];
            v.x = v.x * (g * w.x);
            v.y = v.y * (g * w.y);
            v.z = v.z * (g * w.z);
            v.w = v.w * (g * w.w);
            *at(ck) = v;
        };
#pragma unroll
        for (int k = 0; k < kHeld; ++k) {
            const int ck = threadIdx.x + k * B;
            if (ck < chunks) put(ck, orr[k], grr[k]);
        }
        for (int ck = threadIdx.x + kHeld * B; ck < chunks; ck += B) put(ck, *at(ck), gs[ck]);
        __syncthreads();
    }
};

// The first index of the largest logit (std::max_element, engine.cpp:606-610).
__global__ __launch_bounds__(kNormThreads) void argmax_kernel(const float* __restrict__ x, int n, int* __restrict__ out) {
    __shared__ float bv[kNormThreads / kWave];
    __shared__ int bi[kNormThreads / kWave];
    float best = -INFINITY;
    int index = n;
    for (int i = threadIdx.x; i < n; i += kNormThreads)
        if (x[i] > best || index == n) { best = x[i]; index = i; }
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

// Moves past `count` tokens: step (index into the token list) and position.
__global__ void advance_kernel(int* step, int* position, int count) {
    *step += count;
    *position += count;
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
    float* conv_state = nullptr;  // DeltaNet: [2][DQKV, CK - 1] (copies by position parity)
    float* memory = nullptr;      //           [VH, VD, KD] (column by column)
    float* key_cache = nullptr;   // attention: [capacity, KVH, AD]
    float* value_cache = nullptr;
};

bool engine_config_ok(const q3x_hip_model_config& c, int context) {
    return (c.matrix_type == Q3X_HIP_MATRIX_Q8_0 || c.matrix_type == Q3X_HIP_MATRIX_Q4_0) && c.KD <= 128 &&
           c.VD <= 128 && c.AD <= 256 && c.RD <= 64 && c.RD % 2 == 0 && c.RD <= c.AD && c.CK >= 2 && c.CK <= 8 &&
           c.AH / c.KVH <= kMaxGroup && c.AD % 32 == 0 &&
           c.top_k <= 8 && context >= 1 && context <= 262144;
}

}  // namespace

struct q3x_hip_engine {
    q3x_hip_model_config c{};
    int capacity = 0;
    int chunk = 0;                // rows of a prefill chunk
    int position = 0;             // host mirror of *d_position
    // A forward failed after it had started work on the device: the state
    // may hold part of its tokens.  Forward refuses to run until a reset or
    // a checkpoint restore puts the state back in order.
    bool failed = false;
    int checkpoint_position = 0;
    Mat embedding, lm_head;
    const uint16_t* final_norm = nullptr;
    std::vector<LayerWeights> layers;
    // device memory: one arena
    void* arena = nullptr;
    float *hidden = nullptr, *normalized = nullptr, *branch = nullptr, *logits = nullptr;
    float *qkv = nullptr, *z = nullptr, *a = nullptr, *b = nullptr, *delta_out = nullptr;
    float* delta_gate = nullptr;  // a decode step's norm[j] * silu(z) of the gated RMSNorm, [VH * VD]
    float *query_and_gate = nullptr, *query = nullptr, *gate = nullptr, *key = nullptr, *value = nullptr;
    float *attn_out = nullptr, *scores = nullptr, *ffn_gate = nullptr, *ffn_up = nullptr;
    float *recurrent = nullptr, *checkpoint_recurrent = nullptr, *checkpoint_logits = nullptr;
    size_t recurrent_floats = 0;
    int *d_tokens = nullptr, *d_step = nullptr, *d_position = nullptr, *d_argmax = nullptr;
    void* moe_ws = nullptr;
    size_t moe_ws_bytes = 0;
    // The chunked delta rule's per-(chunk, value head) operands for a chunk
    // of rows (null: the token-by-token scan), and the prefill GEMMs' K-split
    // partial sums, in one scratch region (never in use at once).
    float* delta_ws = nullptr;
    size_t delta_ws_floats = 0;
    void* scratch = nullptr;
    size_t gemm_ws_bytes = 0;
    int* h_tokens = nullptr;  // pinned staging of a forward's counters and tokens
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

// A prefill GEMM's workspace (its K split's partial sums): the engine's
// scratch region, shared with the chunked delta rule's operands (their uses
// never overlap on the engine's one stream).
struct GemmScratch {
    void* p = nullptr;
    size_t bytes = 0;
};

// One matrix applied to `count` rows of x: the matvec for a decode step, the
// prefill GEMM for a chunk.
int apply(const Mat& m, uint32_t type, const float* x, int count, float* y, bool accumulate, hipStream_t s,
          GemmScratch ws = {}) {
    if (count == 1) return q3x_hip_mv(m.w, type, m.rows, m.cols, x, y, accumulate ? 1 : 0, s);
    return q3x_hip_gemm_ws(m.w, type, m.rows, m.cols, x, count, y, accumulate ? 1 : 0, ws.p, ws.bytes, s);
}

// Several matrices of width `cols` applied to the same rows: one multi-matrix
// launch for a decode step (the reference's projection helpers,
// engine.cu:1599-1661), one GEMM each for a chunk.
int apply_group(const Mat* m, float* const* y, int n, uint32_t type, int cols, const float* x, int count,
                hipStream_t s, GemmScratch ws = {}) {
    if (count == 1) {
        q3x_hip_mv_item items[Q3X_HIP_MV_MULTI_MAX];
        for (int i = 0; i < n; ++i) items[i] = q3x_hip_mv_item{m[i].w, m[i].rows, y[i], 0};
        return q3x_hip_mv_multi(items, n, type, cols, x, s);
    }
    for (int i = 0; i < n; ++i) {
        const int rc = q3x_hip_gemm_ws(m[i].w, type, m[i].rows, cols, x, count, y[i], 0, ws.p, ws.bytes, s);
        if (rc) return rc;
    }
    return Q3X_HIP_OK;
}

// A decode step's matvec of the matrices m[0..n) (same width `cols`) over
// x, with `in` staging x into LDS (a norm or SwiGLU applied on the way in):
// one launch of the pipelined kernel; add[i]: y[i] += W x.  Returns
// Q3X_HIP_ENOTSUP before launching anything where that kernel does not take
// the shape (x too long for LDS, unaligned rows); the caller then runs the
// separate kernels.
template <class In>
int mv_staged(const Mat* m, float* const* y, const bool* add, int n, uint32_t type, int cols, const float* x,
              const In& in, hipStream_t s, uint32_t silu_mask = 0) {
    const int bpr = cols / kBlock;
    const size_t row_bytes = static_cast<size_t>(bpr) * block_bytes(type);
    if (row_bytes % 16 != 0 || !aligned(x, 16) || n < 1 || n > MultiRows::kMax) return Q3X_HIP_ENOTSUP;
    MultiRows map{};
    map.count = n;
    map.row_bytes = row_bytes;
    map.x = x;
    map.silu_mask = silu_mask;
    int total = 0;
    for (int i = 0; i < n; ++i) {
        if (!aligned(m[i].w, 16) || m[i].cols != cols) return Q3X_HIP_ENOTSUP;
        total += m[i].rows;
        map.w[i] = static_cast<const uint8_t*>(m[i].w);
        map.y[i] = y[i];
        map.end[i] = total;
        if (add[i]) map.accumulate_mask |= 1u << i;
    }
    for (int i = n; i < MultiRows::kMax; ++i) {
        map.w[i] = map.w[0];
        map.y[i] = map.y[0];
        map.end[i] = total;
    }
    return type == Q3X_HIP_MATRIX_Q8_0 ? launch_pipe_for<Q3X_HIP_MATRIX_Q8_0>(map, total, bpr, s, in)
                                       : launch_pipe_for<Q3X_HIP_MATRIX_Q4_0>(map, total, bpr, s, in);
}

// Enqueues `count` tokens (tokens[*d_step ..] at *d_position ..) through
// every layer; the logits of the last one when `logits`; then advances the
// step and position by count.  count 1 is the decode step the graphs
// capture; count > 1 (at most kChunk) a prefill chunk.
int enqueue(q3x_hip_engine& e, int count, bool logits) {
    const q3x_hip_model_config& c = e.c;
    hipStream_t s = e.stream;
    const int DO = c.VH * c.VD, DQKV = 2 * c.KH * c.KD + DO;
    const uint32_t type = c.matrix_type;
    const GemmScratch gemm_ws{e.scratch, e.gemm_ws_bytes};
    const dim3 eg((c.H + 255) / 256, count);
    if (type == Q3X_HIP_MATRIX_Q8_0)
        hipLaunchKernelGGL(embed_kernel<Q3X_HIP_MATRIX_Q8_0>, eg, dim3(256), 0, s,
                           static_cast<const uint8_t*>(e.embedding.w), c.H, e.d_tokens, e.d_step, e.hidden);
    else
        hipLaunchKernelGGL(embed_kernel<Q3X_HIP_MATRIX_Q4_0>, eg, dim3(256), 0, s,
                           static_cast<const uint8_t*>(e.embedding.w), c.H, e.d_tokens, e.d_step, e.hidden);
    int rc = launch_status();
    // A decode step forms each norm and SwiGLU inside the matvec that reads
    // it, and adds an MoE layer's output to hidden directly; a chunk (or a
    // shape those launches do not take) runs them as kernels of their own.
    const bool step = count == 1;
    const bool no_add[4] = {false, false, false, false};
    bool pending = false;  // an MoE output in `branch` still to be added to hidden
    for (int i = 0; i < c.N && rc == Q3X_HIP_OK; ++i) {
        const LayerWeights& L = e.layers[i];
        const int nproj = L.attention ? 3 : 4;
        const Mat proj[4] = {L.attention ? L.q : L.qkv, L.attention ? L.k : L.z, L.attention ? L.v : L.a, L.b};
        float* const proj_out[4] = {L.attention ? e.query_and_gate : e.qkv, L.attention ? e.key : e.z,
                                    L.attention ? e.value : e.a, e.b};
        rc = Q3X_HIP_ENOTSUP;
        if (step && !pending && aligned(L.input_norm, 8))
            rc = mv_staged(proj, proj_out, no_add, nproj, type, c.H, e.hidden, NormInput{L.input_norm}, s);
        if (rc == Q3X_HIP_ENOTSUP) {
            hipLaunchKernelGGL(rms_kernel, dim3(count), dim3(kNormThreads), 0, s, e.hidden,
                               pending ? e.branch : nullptr, L.input_norm, c.H, e.normalized);
            rc = apply_group(proj, proj_out, nproj, type, c.H, e.normalized, count, s, gemm_ws);
        }
        if (rc) break;
        if (!L.attention) {
            if (count == 1) {
                // The conv of the step's channels runs inside the delta rule;
                // the gated norm inside the out projection's staging.
                hipLaunchKernelGGL(delta_step_kernel, dim3(c.VH * kScanSlices), dim3(kScanThreads), 0, s, e.qkv, e.a,
                                   e.b, e.z, L.alog, L.dt, L.norm, L.memory, e.delta_out, e.delta_gate, L.conv,
                                   L.conv_state, e.d_position, c.CK, c.KH, c.VH, c.KD, c.VD);
                const bool add_out[1] = {true};
                float* const out_y[1] = {e.hidden};
                rc = c.VD % 4 == 0 && c.VH <= 256
                         ? mv_staged(&L.out, out_y, add_out, 1, type, DO, e.delta_out,
                                     GatedNormInput{e.delta_gate, c.VD}, s)
                         : Q3X_HIP_ENOTSUP;
                if (rc == Q3X_HIP_ENOTSUP) {
                    hipLaunchKernelGGL(delta_norm_kernel, dim3(c.VH, 1), dim3(128), 0, s, e.delta_out, e.z, L.norm,
                                       c.VH, c.VD);
                    rc = apply(L.out, type, e.delta_out, count, e.hidden, true, s, gemm_ws);
                }
            } else {
                hipLaunchKernelGGL(delta_conv_kernel<16>, dim3((DQKV + kConvThreads / 16 - 1) / (kConvThreads / 16)),
                                   dim3(kConvThreads), 0, s, e.qkv, L.conv, L.conv_state, e.d_position, DQKV, c.CK,
                                   count);
                hipLaunchKernelGGL(delta_prep_kernel, dim3(c.KH, count), dim3(128), 0, s, e.qkv, e.a, e.b, L.alog,
                                   L.dt, c.KH, c.VH, c.KD, c.VD);
                if (e.delta_ws) {
                    // The recurrence in chunks on the matrix cores.
                    hipLaunchKernelGGL(delta_chunk_prep_kernel, dim3((count + kDeltaChunk - 1) / kDeltaChunk, c.VH),
                                       dim3(kDeltaPrepThreads), 0, s, e.qkv, e.a, e.b, e.delta_ws, c.KH, c.VH, c.KD,
                                       c.VD, count);
                    hipLaunchKernelGGL(delta_chunk_scan_kernel, dim3(c.VH * (c.VD / 32)),
                                       dim3(kDeltaScanWaves * kWave), 0, s, e.qkv, e.delta_ws, L.memory,
                                       e.delta_out, c.KH, c.VH, c.KD, c.VD, count);
                } else {
                    hipLaunchKernelGGL(delta_scan_kernel, dim3(c.VH * kScanSlices), dim3(kScanThreads), 0, s,
                                       e.qkv, e.a, e.b, L.memory, e.delta_out, c.KH, c.VH, c.KD, c.VD, count);
                }
                hipLaunchKernelGGL(delta_norm_kernel, dim3(c.VH, count), dim3(128), 0, s, e.delta_out, e.z, L.norm,
                                   c.VH, c.VD);
                rc = apply(L.out, type, e.delta_out, count, e.hidden, true, s, gemm_ws);
            }
        } else {
            hipLaunchKernelGGL(attention_prep_kernel, dim3(c.AH + c.KVH, count), dim3(kHeadThreads), 0, s,
                               e.query_and_gate, e.key, e.value, L.qnorm, L.knorm, e.d_position, e.query, e.gate,
                               L.key_cache, L.value_cache, c.AH, c.KVH, c.AD, c.RD);
            if (count == 1) {
                auto attend = c.AH / c.KVH <= 4 ? attention_kernel<4> : attention_kernel<8>;
                hipLaunchKernelGGL(attend, dim3(c.KVH * kAttnSplits), dim3(kHeadThreads), 0, s, e.query,
                                   L.key_cache, L.value_cache, e.d_position, e.scores, c.AH, c.KVH, c.AD,
                                   kAttnSplits);
                hipLaunchKernelGGL(attention_combine_kernel, dim3(c.AH, (c.AD + kCombCols - 1) / kCombCols, 1),
                                   dim3(kHeadThreads), 0, s, e.scores, e.gate, e.attn_out, c.AH, c.AD);
            } else {
                const int subs = (c.AH / c.KVH + kFlashWaves - 1) / kFlashWaves;
                hipLaunchKernelGGL(attention_prefill_kernel, dim3(c.KVH * subs, (count + kFlashQ - 1) / kFlashQ),
                                   dim3(kFlashWaves * kWave), kFlashLds, s, e.query, e.gate, L.key_cache,
                                   L.value_cache, e.d_position, e.attn_out, c.AH, c.KVH, c.AD, count);
            }
            rc = apply(L.o, type, e.attn_out, count, e.hidden, true, s, gemm_ws);
        }
        if (rc) break;
        if (c.experts) {
            // Decode: the post-attention norm inside the router and expert
            // launches, the layer's output added to the residual in place.
            rc = step ? moe_layer_decode_add(L.moe, e.hidden, L.post_norm, e.hidden, e.moe_ws, e.moe_ws_bytes, s)
                      : Q3X_HIP_ENOTSUP;
            pending = rc == Q3X_HIP_ENOTSUP;
            if (pending) {
                hipLaunchKernelGGL(rms_kernel, dim3(count), dim3(kNormThreads), 0, s, e.hidden, nullptr,
                                   L.post_norm, c.H, e.normalized);
                rc = q3x_hip_moe_layer(&L.moe, e.normalized, count, e.branch, nullptr, nullptr, e.moe_ws,
                                       e.moe_ws_bytes, s);
            }
        } else {
            const Mat gate_up[2] = {L.gate, L.up};
            float* const ffn[2] = {e.ffn_gate, e.ffn_up};
            // A decode step stores silu(gate) (matrix 0) for the down
            // launch's SwiGLUInput.
            rc = step && aligned(L.post_norm, 8)
                     ? mv_staged(gate_up, ffn, no_add, 2, type, c.H, e.hidden, NormInput{L.post_norm}, s, 1u)
                     : Q3X_HIP_ENOTSUP;
            const bool silu_stored = rc == Q3X_HIP_OK;
            bool swiglu_done = false;  // ffn_gate holds silu(gate) * up
            if (rc == Q3X_HIP_ENOTSUP) {
                hipLaunchKernelGGL(rms_kernel, dim3(count), dim3(kNormThreads), 0, s, e.hidden, nullptr,
                                   L.post_norm, c.H, e.normalized);
                // A chunk: gate and up as one GEMM with the SwiGLU in its
                // epilogue (one pass over h instead of three).
                rc = count > 1 ? gate_up_swiglu(L.gate.w, L.up.w, type, c.I, c.H, e.normalized, count, e.ffn_gate, s)
                               : Q3X_HIP_ENOTSUP;
                swiglu_done = rc == Q3X_HIP_OK;
                if (rc == Q3X_HIP_ENOTSUP) rc = apply_group(gate_up, ffn, 2, type, c.H, e.normalized, count, s, gemm_ws);
            }
            if (rc) break;
            const bool add = true;
            float* const residual = e.hidden;
            rc = silu_stored ? mv_staged(&L.down, &residual, &add, 1, type, c.I, e.ffn_gate, SwiGLUInput{e.ffn_up}, s)
                             : Q3X_HIP_ENOTSUP;
            if (rc == Q3X_HIP_ENOTSUP) {
                const int n = count * c.I;
                if (swiglu_done) {
                } else if (silu_stored) {  // silu(gate) already: x = gate * up
                    hipLaunchKernelGGL(product_kernel, dim3((n + 255) / 256), dim3(256), 0, s, e.ffn_gate, e.ffn_up, n);
                } else {
                    hipLaunchKernelGGL(swiglu_kernel, dim3((n + 255) / 256), dim3(256), 0, s, e.ffn_gate, e.ffn_up, n);
                }
                rc = apply(L.down, type, e.ffn_gate, count, e.hidden, true, s, gemm_ws);
            }
            pending = false;
        }
        if (rc == Q3X_HIP_OK) rc = launch_status();
    }
    if (rc) return rc;
    if (logits) {
        // The last row only: its residual, final norm and lm_head.
        const size_t last = static_cast<size_t>(count - 1) * c.H;
        rc = Q3X_HIP_ENOTSUP;
        if (step && !pending && aligned(e.final_norm, 8))
            rc = mv_staged(&e.lm_head, &e.logits, no_add, 1, type, c.H, e.hidden, NormInput{e.final_norm}, s);
        if (rc == Q3X_HIP_ENOTSUP) {
            hipLaunchKernelGGL(rms_kernel, dim3(1), dim3(kNormThreads), 0, s, e.hidden + last,
                               pending ? e.branch + last : nullptr, e.final_norm, c.H, e.normalized);
            rc = q3x_hip_mv(e.lm_head.w, type, e.lm_head.rows, e.lm_head.cols, e.normalized, e.logits, 0, s);
        }
        if (rc) return rc;
    }
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, e.d_step, e.d_position, count);
    return launch_status();
}

int capture(q3x_hip_engine& e, bool logits) {
    hipGraph_t g = nullptr;
    if (hipStreamBeginCapture(e.stream, hipStreamCaptureModeThreadLocal) != hipSuccess) return Q3X_HIP_ERUNTIME;
    const int rc = enqueue(e, 1, logits);
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
                                     int chunk, q3x_hip_engine** engine, const char** error) {
    if (!config || !weights || !engine || chunk < 0) return Q3X_HIP_EINVAL;
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
    const size_t conv = 2 * static_cast<size_t>(DQKV) * (c.CK - 1);
    const size_t memory = static_cast<size_t>(c.VH) * c.KD * c.VD;
    const size_t cache = static_cast<size_t>(context) * KVW;
    const int delta_layers = c.N - c.N / c.AI;
    e->recurrent_floats = static_cast<size_t>(delta_layers) * (conv + memory);
    e->chunk = std::min(context, chunk > 0 ? chunk : kChunk);
    const size_t R = static_cast<size_t>(e->chunk);  // rows of a chunk
    if (c.experts)
        e->moe_ws_bytes = std::max(q3x_hip_moe_layer_workspace_bytes(&e->layers[0].moe, 1),
                                   q3x_hip_moe_layer_workspace_bytes(&e->layers[0].moe, static_cast<int>(R)));
    e->token_capacity = context;
    // The chunked delta rule takes key and value heads of whole 32-wide
    // blocks (every model of the family: 128); others run the token scan.
    if (c.VH > 0 && c.KD % 32 == 0 && c.VD % 32 == 0)
        e->delta_ws_floats = (R + kDeltaChunk - 1) / kDeltaChunk * c.VH * static_cast<size_t>(kDeltaChunkFloats);
    // The prefill GEMMs' K splits: the most any of the chunk's GEMMs asks
    // for at any row count up to a chunk (a call given less runs unsplit),
    // within kGemmScratchMax.
    if (R > 1) {
        auto need = [&](const Mat& m) {
            size_t most = 0;
            if (!m.w) return most;
            for (size_t n = 64; n < R + 64; n += 64) {
                const int count = static_cast<int>(std::min(n, R));
                most = std::max(most, q3x_hip_gemm_workspace_bytes(c.matrix_type, m.rows, m.cols, count));
            }
            return most;
        };
        for (const LayerWeights& L : e->layers)
            for (const Mat* m : {&L.qkv, &L.z, &L.a, &L.b, &L.out, &L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down})
                e->gemm_ws_bytes = std::max(e->gemm_ws_bytes, need(*m));
        if (e->gemm_ws_bytes > kGemmScratchMax) e->gemm_ws_bytes = kGemmScratchMax;
    }
    // One arena: the work rows of a chunk, the recurrent state and its
    // checkpoint, the KV caches, the logits, the token list and counters.
    // plan(base) carves it; plan(nullptr) only measures it.
    auto plan = [&](uint8_t* base) -> size_t {
        size_t at = 0;
        auto take = [&](size_t n, size_t size) {
            uint8_t* p = base ? base + at : nullptr;
            at += (n * size + 255) / 256 * 256;
            return p;
        };
        auto f = [&](size_t n) { return reinterpret_cast<float*>(take(n, 4)); };
        e->hidden = f(R * c.H);
        e->normalized = f(R * c.H);
        e->branch = f(R * c.H);
        e->logits = f(c.V);
        e->qkv = f(R * DQKV);
        e->z = f(R * DO);
        e->a = f(R * c.VH);
        e->b = f(R * c.VH);
        e->delta_out = f(R * DO);
        e->delta_gate = f(DO);
        e->query_and_gate = f(R * 2 * AS);
        e->query = f(R * AS);
        e->gate = f(R * AS);
        e->key = f(R * KVW);
        e->value = f(R * KVW);
        e->attn_out = f(R * AS);
        e->scores = f(static_cast<size_t>(c.AH) * kAttnSplits * (c.AD + 2));
        e->ffn_gate = f(R * c.I);
        e->ffn_up = f(R * c.I);
        e->recurrent = f(e->recurrent_floats);
        e->checkpoint_recurrent = f(e->recurrent_floats);
        e->checkpoint_logits = f(c.V);
        float* rec = e->recurrent;
        for (int i = 0; i < c.N; ++i) {
            LayerWeights& L = e->layers[i];
            if (!L.attention) {
                L.conv_state = rec;
                if (rec) rec += conv;
                L.memory = rec;
                if (rec) rec += memory;
            } else {
                L.key_cache = f(cache);
                L.value_cache = f(cache);
            }
        }
        // [step, position, tokens...]: one copy from the pinned staging
        // sets a forward's counters and tokens.
        e->d_step = reinterpret_cast<int*>(take(2 + static_cast<size_t>(e->token_capacity), 4));
        e->d_position = e->d_step + 1;
        e->d_tokens = e->d_step + 2;
        e->d_argmax = reinterpret_cast<int*>(take(1, 4));
        e->moe_ws = e->moe_ws_bytes ? take(e->moe_ws_bytes, 1) : nullptr;
        const size_t scratch = std::max(e->delta_ws_floats * sizeof(float), e->gemm_ws_bytes);
        e->scratch = scratch ? take(scratch, 1) : nullptr;
        e->delta_ws = e->delta_ws_floats ? static_cast<float*>(e->scratch) : nullptr;
        return at;
    };
    const size_t total = plan(nullptr);
    int rc = Q3X_HIP_OK;
    const hipError_t status = hipMalloc(&e->arena, total);
    if (status != hipSuccess) {
        (void)hipGetLastError();
        e->arena = nullptr;
        set_error(error, "HIP engine state does not fit in device memory");
        rc = Q3X_HIP_ERUNTIME;
    }
    if (rc == Q3X_HIP_OK) {
        plan(static_cast<uint8_t*>(e->arena));
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(attention_prefill_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(kFlashLds)) != hipSuccess ||
            hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess ||
            hipHostMalloc(reinterpret_cast<void**>(&e->h_tokens), sizeof(int) * (2 + e->token_capacity),
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
        rc = enqueue(*e, 1, true);
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
    e->failed = false;
    return Q3X_HIP_OK;
}

namespace {

// Work of a forward may already be queued when a later step fails (a prefill
// chunk after the first, the decode graph, the wait for the stream): let the
// queued work end, and refuse further forwards until the state is reset,
// where the reference would abort.
int forward_failed(q3x_hip_engine& e, int rc) {
    (void)hipStreamSynchronize(e.stream);
    (void)hipGetLastError();
    e.failed = true;
    return rc;
}

}  // namespace

extern "C" int q3x_hip_engine_forward(q3x_hip_engine* e, const int* tokens, int count, int compute_logits) {
    if (!e || !tokens || count <= 0) return Q3X_HIP_EINVAL;
    if (e->failed) return Q3X_HIP_ESTATE;
    if (count > e->capacity - e->position) return Q3X_HIP_EINVAL;
    for (int i = 0; i < count; ++i)
        if (tokens[i] < 0 || tokens[i] >= e->c.V) return Q3X_HIP_EINVAL;
    e->h_tokens[0] = 0;  // step: index of the next token in the list
    e->h_tokens[1] = e->position;
    for (int i = 0; i < count; ++i) e->h_tokens[2 + i] = tokens[i];
    // Nothing has reached the device if the token copy cannot be queued.
    if (hipMemcpyAsync(e->d_step, e->h_tokens, sizeof(int) * (2 + count), hipMemcpyHostToDevice, e->stream) !=
        hipSuccess)
        return Q3X_HIP_ERUNTIME;
    if (count == 1) {
        hipGraphExec_t& g = e->graph[compute_logits ? 1 : 0];
        if (!g) {
            // A capture runs nothing on the device: on failure the state, the
            // KV cache and the position are as they were (the token copy
            // queued above is rewritten by the next forward), so the engine
            // stays usable and the error is returned as it is.
            const int rc = capture(*e, compute_logits != 0);
            if (rc) {
                (void)hipStreamSynchronize(e->stream);
                (void)hipGetLastError();
                return rc;
            }
        }
        if (hipGraphLaunch(g, e->stream) != hipSuccess) return forward_failed(*e, Q3X_HIP_ERUNTIME);
    } else {
        for (int done = 0; done < count;) {
            const int n = std::min(e->chunk, count - done);
            const int rc = enqueue(*e, n, compute_logits && done + n == count);
            if (rc) return forward_failed(*e, rc);
            done += n;
        }
    }
    if (count == 1) {
        // A decode step lasts milliseconds: poll for its end rather than
        // sleep in the runtime's wait, which wakes tens of microseconds late.
        hipError_t q;
        while ((q = hipStreamQuery(e->stream)) == hipErrorNotReady) {
        }
        if (q != hipSuccess) return forward_failed(*e, Q3X_HIP_ERUNTIME);
    } else if (hipStreamSynchronize(e->stream) != hipSuccess) {
        return forward_failed(*e, Q3X_HIP_ERUNTIME);
    }
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
    e->failed = false;
    return Q3X_HIP_OK;
}

extern "C" int q3x_hip_engine_position(const q3x_hip_engine* e) { return e ? e->position : -1; }
