// rows.h -- row maps for the matvec kernels: where virtual row r of a launch
// lives, which activations it reads, and where its result goes.
#pragma once

#include "common.h"

namespace q3x {

// The reference's sigmoid / silu (engine.cpp:187-191): the branch keeps the
// exponential's argument non-positive.
__device__ __forceinline__ float sigmoid_ref(float x) {
    if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
    const float e = expf(x);
    return e / (1.0f + e);
}
__device__ __forceinline__ float silu_ref(float x) { return x * sigmoid_ref(x); }

// One dense matrix W[rows, cols]: y[r] = W[r] x, or y[r] += W[r] x when
// ACCUMULATE (compile-time, so the plain product never reads y).
template <bool ACCUMULATE>
struct DenseRows {
    static constexpr bool kSharedInput = true;  // every row reads x
    static constexpr bool kSwiGLUPairs = false;  // rows are stored one by one
    const uint8_t* w;
    size_t row_bytes;
    const float* x;
    float* y;
    __device__ const uint8_t* row(int r) const { return w + static_cast<size_t>(r) * row_bytes; }
    __device__ const uint8_t* any() const { return w; }  // a valid address of the matrix
    __device__ const float* input(int) const { return x; }
    // Value the result is added to.
    __device__ float previous(int r) const { return ACCUMULATE ? y[r] : 0.0f; }
    __device__ void store(int r, float v) const { y[r] = v; }
    __host__ int matrices() const { return 1; }
    __host__ void plan_waves(int) {}
    __device__ const DenseRows& for_wave(int&, int&, int&) const { return *this; }
};

// One dense matrix chosen at run time (a wave's share of a multi-matrix
// launch): y[r] = W[r] x, or y[r] += W[r] x when `accumulate`.
struct OneMatrix {
    static constexpr bool kSharedInput = true;
    static constexpr bool kSwiGLUPairs = false;
    const uint8_t* w;  // null: every row reads as zeros (an expert id out of range)
    size_t row_bytes;
    const float* x;
    float* y;
    bool accumulate;
    const uint8_t* any_w;  // a valid address for empty buffer ranges
    bool silu = false;     // store silu(v) (the gate half of a decode step's SwiGLU)
    __device__ const uint8_t* row(int r) const { return w ? w + static_cast<size_t>(r) * row_bytes : nullptr; }
    __device__ const uint8_t* any() const { return any_w; }
    __device__ const float* input(int) const { return x; }
    __device__ float previous(int r) const { return accumulate ? load_global(y + r) : 0.0f; }
    __device__ void store(int r, float v) const { store_global(y + r, silu ? silu_ref(v) : v); }
};

// Up to Q3X_HIP_MV_MULTI_MAX matrices of one type and width that read the
// same x.  Matrix i holds virtual rows [end[i-1], end[i]) and owns the waves
// [wave_end[i-1], wave_end[i]) of the launch (in proportion to its rows, set
// by plan_waves once the launch's wave count is known), so a wave looks its
// matrix up once, at the start, and then streams it like a dense matrix.
struct MultiRows {
    static constexpr bool kSharedInput = true;
    static constexpr int kMax = Q3X_HIP_MV_MULTI_MAX;
    const uint8_t* w[kMax];
    float* y[kMax];
    int end[kMax];
    int wave_end[kMax];
    int count;
    uint32_t accumulate_mask;
    // Matrices whose rows store silu(W x) instead of W x: a decode step's
    // gate, so that the down projection's input staging forms
    // silu(gate) * up with one multiply per value instead of every
    // workgroup evaluating silu over the whole row (engine.cpp:371-376).
    uint32_t silu_mask = 0;
    size_t row_bytes;
    const float* x;

    __host__ __device__ int rows_of(int i) const { return end[i] - (i ? end[i - 1] : 0); }
    __host__ int matrices() const { return count; }

    // Waves per matrix for a launch of GW waves (GW >= count): one each, then
    // the rest in proportion to the rows, the remainder to the matrices with
    // the most rows per wave.
    __host__ void plan_waves(int GW) {
        const long long total = end[count - 1];
        int waves[kMax];
        int used = 0;
        for (int i = 0; i < count; ++i) {
            waves[i] = 1 + static_cast<int>((static_cast<long long>(GW - count) * rows_of(i)) / total);
            used += waves[i];
        }
        while (used < GW) {
            int best = 0;
            for (int i = 1; i < count; ++i)
                if (static_cast<long long>(rows_of(i)) * waves[best] > static_cast<long long>(rows_of(best)) * waves[i])
                    best = i;
            ++waves[best];
            ++used;
        }
        int acc = 0;
        for (int i = 0; i < kMax; ++i) {
            acc += i < count ? waves[i] : 0;
            wave_end[i] = acc;
        }
    }

    // The matrix of wave gw; gw, GW and nrows become that matrix's own wave
    // index, wave count and row count.  Unrolled over the fixed maximum with
    // compile-time indices, so the table stays in scalar registers.
    __device__ OneMatrix for_wave(int& gw, int& GW, int& nrows) const {
        int k = 0;
#pragma unroll
        for (int i = 1; i < kMax; ++i)
            if (i < count && gw >= wave_end[i - 1]) k = i;
        const uint8_t* wk = nullptr;
        float* yk = nullptr;
        int first_wave = 0, first_row = 0, last_wave = 0, last_row = 0;
#pragma unroll
        for (int i = 0; i < kMax; ++i) {
            // Opaque scalar copies: keeps the compiler from turning this
            // select chain into an indexed access of a private copy of the
            // table (scratch memory and divergent pointers).
            const uint8_t* wi = w[i];
            float* yi = y[i];
            int fw = i ? wave_end[i - 1] : 0, fr = i ? end[i - 1] : 0, lw = wave_end[i], lr = end[i];
            asm volatile("" : "+s"(wi), "+s"(yi), "+s"(fw), "+s"(fr), "+s"(lw), "+s"(lr));
            if (i == k) {
                wk = wi;
                yk = yi;
                first_wave = fw;
                first_row = fr;
                last_wave = lw;
                last_row = lr;
            }
        }
        gw -= first_wave;
        GW = last_wave - first_wave;
        nrows = last_row - first_row;
        return OneMatrix{wk, row_bytes, x, yk, ((accumulate_mask >> k) & 1u) != 0, wk, ((silu_mask >> k) & 1u) != 0};
    }
};

// The experts one token selected, viewed as one tall matrix for the gate_up
// matvec of a decode step: virtual row r = slot * rows_per_expert + j is row
// j of expert ids[slot] in the pool [experts, rows_per_expert, cols], and
// every slot reads x.  The launch's waves are split evenly over the slots
// (plan_waves), so a wave reads its slot's expert id once, at the start.  An
// id outside [0, experts) reads as zeros (the reference CUDA kernels skip such
// slots, engine.cu:1198, 1235).  The result of virtual row r goes to y[r].
struct ExpertRows {
    static constexpr bool kSharedInput = true;
    static constexpr int kMaxSlots = 9;  // top_k <= 8, plus a shared expert
    const uint8_t* pool;
    size_t expert_bytes;
    size_t row_bytes;
    int rows_per_expert;
    int experts;
    const int* ids;
    int slots;
    const float* x;
    float* y;
    int wave_end[kMaxSlots];

    __host__ int matrices() const { return slots; }
    __host__ void plan_waves(int GW) {
        for (int s = 0; s < kMaxSlots; ++s)
            wave_end[s] = static_cast<int>((static_cast<long long>(GW) * (s < slots ? s + 1 : slots)) / slots);
    }
    // The slot of wave gw; gw and GW become the wave's index and the wave
    // count within that slot.
    __device__ int slot_of_wave(int& gw, int& GW) const {
        int s = 0;
#pragma unroll
        for (int i = 1; i < kMaxSlots; ++i)
            if (i < slots && gw >= wave_end[i - 1]) s = i;
        int first = 0, last = wave_end[0];
#pragma unroll
        for (int i = 1; i < kMaxSlots; ++i) {
            int fw = wave_end[i - 1], lw = wave_end[i];
            asm volatile("" : "+s"(fw), "+s"(lw));  // keep the table in scalar registers
            if (i == s) { first = fw; last = lw; }
        }
        gw -= first;
        GW = last - first;
        return s;
    }
    // Expert matrix of slot s (null when its id is out of range), the ids
    // read from `src` (ids, or a launch's own routing in LDS).
    __device__ const uint8_t* expert_of_slot(int s, const int* src) const {
        const int e = __builtin_amdgcn_readfirstlane(src[s]);
        return e >= 0 && e < experts ? pool + static_cast<size_t>(e) * expert_bytes : nullptr;
    }
    __device__ const uint8_t* expert_of_slot(int s) const { return expert_of_slot(s, ids); }
    __device__ OneMatrix for_wave(int& gw, int& GW, int& nrows) const {
        const int s = slot_of_wave(gw, GW);
        nrows = rows_per_expert;
        return OneMatrix{expert_of_slot(s), row_bytes, x, y + static_cast<size_t>(s) * rows_per_expert, false, pool};
    }
};

// A wave's share of ExpertGateUpRows: the gate rows and up rows of one
// expert (rows [0, I) and [I, 2I) of its gate_up matrix, or the shared
// expert's two matrices), numbered so that the two row iterations of a step
// (virtual rows v and v + GW, v = gw + 2b * GW) are gate row q and up row q of
// the same q = gw + b * GW; the step stores h[q] = silu(gate . x) * (up . x)
// (engine.cpp:413-416, 422-425).  Pairs q >= I read zeros and store nothing.
struct GateUpPairs {
    static constexpr bool kSharedInput = true;
    static constexpr bool kSwiGLUPairs = true;
    const uint8_t* gate;  // null: expert id out of range (rows read as zeros)
    const uint8_t* up;
    size_t row_bytes;
    const float* x;
    float* h;
    int I;
    int GW;  // the waves of this slot: the stride of the wave's rows
    const uint8_t* any_w;
    __device__ int pair(int v) const { return v % GW + (v / GW / 2) * GW; }
    __device__ const uint8_t* row(int v) const {
        const int q = pair(v);
        // gate or up by arithmetic, not a select of the two members (which
        // the compiler turns into an indexed load from a private copy).
        const uintptr_t g = reinterpret_cast<uintptr_t>(gate), u = reinterpret_cast<uintptr_t>(up);
        const uint8_t* base = reinterpret_cast<const uint8_t*>(g + static_cast<uintptr_t>((v / GW) % 2) * (u - g));
        if (!base || q >= I) return nullptr;
        return base + static_cast<size_t>(q) * row_bytes;
    }
    __device__ const uint8_t* any() const { return any_w; }
    __device__ const float* input(int) const { return x; }
    __device__ void store_pair(int v_gate, float gate_dot, float up_dot) const {
        const int q = pair(v_gate);
        if (q < I) store_global(h + q, silu_ref(gate_dot) * up_dot);
    }
};

// The decode step's gate_up matvec with SwiGLU applied: the experts of
// ExpertRows (waves split evenly over the slots), each slot's result
// h[slot * I + q] = silu(G_e[q] . x) * (U_e[q] . x).  With shared_gate set,
// the last slot is the shared expert (shared_gate / shared_up, shared_I <= I
// rows).  For the pipelined kernel with one row group of 64 lanes and two row
// iterations per step.
struct ExpertGateUpRows : ExpertRows {
    int I;
    const uint8_t* shared_gate;
    const uint8_t* shared_up;
    int shared_I;
    __device__ GateUpPairs for_wave(int& gw, int& GW, int& nrows) const { return for_wave(gw, GW, nrows, ids); }
    __device__ GateUpPairs for_wave(int& gw, int& GW, int& nrows, const int* src) const {
        const int s = slot_of_wave(gw, GW);
        const bool shared = shared_gate && s == slots - 1;
        const int rows = shared ? shared_I : I;
        // Virtual rows: two per pair, every wave the same number of steps.
        nrows = 2 * GW * ((rows + GW - 1) / GW);
        float* h = y + static_cast<size_t>(s) * I;
        if (shared) return GateUpPairs{shared_gate, shared_up, row_bytes, x, h, rows, GW, pool};
        const uint8_t* w = expert_of_slot(s, src);
        const uint8_t* up = w ? w + static_cast<size_t>(I) * row_bytes : nullptr;
        return GateUpPairs{w, up, row_bytes, x, h, rows, GW, pool};
    }
};

}  // namespace q3x
