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
};

// The experts one token selected, viewed as one tall matrix: virtual row
// r = slot * rows_per_expert + j is row j of expert ids[slot] in the pool
// [experts, rows_per_expert, cols].  An id outside [0, experts) yields a
// null row, which the kernels read as zeros (the reference CUDA kernels skip
// such slots, engine.cu:1198, 1235).  SHARED: every slot reads x (gate_up);
// otherwise slot s reads x + s * x_slot_stride (down).  The result of
// virtual row r goes to y[r].
template <bool SHARED>
struct ExpertRows {
    static constexpr bool kSharedInput = SHARED;
    const uint8_t* pool;
    size_t expert_bytes;
    size_t row_bytes;
    int rows_per_expert;
    int experts;
    const int* ids;
    const float* x;
    size_t x_slot_stride;
    float* y;
    __device__ int slot(int r) const { return r / rows_per_expert; }
    __device__ const uint8_t* row(int r) const {
        const int s = slot(r);
        const int e = ids[s];
        if (e < 0 || e >= experts) return nullptr;
        return pool + static_cast<size_t>(e) * expert_bytes +
               static_cast<size_t>(r - s * rows_per_expert) * row_bytes;
    }
    __device__ const uint8_t* any() const { return pool; }
    __device__ const float* input(int r) const { return SHARED ? x : x + slot(r) * x_slot_stride; }
    __device__ float previous(int) const { return 0.0f; }
    __device__ void store(int r, float v) const { y[r] = v; }
};

}  // namespace q3x
