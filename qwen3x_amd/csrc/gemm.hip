// gemm.hip -- q3x_hip_gemm: dense prefill GEMM Y[count, rows] (+)= X W^T
// with Q8_0 / Q4_0 weights: FP32 activations split exactly into three bf16
// parts on the bf16 matrix cores (gemm_x3.h).
//
// Replaces the reference's batch_mv (arch/cuda/engine.cu:1568-1597), whose Q8
// path is an FP32 SIMT kernel (batch_mv_q8_kernel :761, 64 rows x 128 tokens
// per CTA) and which has no Q4_0 GEMM (it asserts, :1580).
#include "gemm.h"
#include "gemm_x3.h"
#include "matvec.h"

namespace q3x {

// Token rows X[count, cols] against one weight matrix.
struct DenseGemm {
    static constexpr bool kLinearGrid = true;
    static constexpr bool kPairedColumns = false;
    static constexpr bool kPartialTiles = false;  // only the last token tile is short
    int tiles_x;  // weight-row tiles of the launch
    const float* X;
    int cols;
    int count;
    const uint8_t* w;
    size_t row_bytes;
    float* Y;
    int rows;
    bool accumulate;
    int ksplit = 1;         // units per tile over K (set by the launch)
    float* part = nullptr;  // their partial sums (caller's workspace)
    __device__ bool tile(int ty, int bm, GemmTile& t) const {
        t.m0 = ty * bm;
        t.mcount = min(bm, count - t.m0);
        t.group = 0;
        return t.mcount > 0;
    }
    __device__ const float* a_row(const GemmTile& t, int m) const {
        return X + static_cast<size_t>(t.m0 + m) * cols;
    }
    __device__ const uint8_t* b_row(const GemmTile&, int n) const {
        return w + static_cast<size_t>(n) * row_bytes;
    }
    __device__ void store(const GemmTile& t, int m, int n, float v) const {
        float* p = Y + static_cast<size_t>(t.m0 + m) * rows + n;
        if (accumulate) *p += v;
        else *p = v;
    }
    __device__ void store_pair(const GemmTile&, int, int, float, float) const {}
};

}  // namespace q3x

using namespace q3x;

namespace {

int gemm(const void* w, uint32_t type, int rows, int cols, const float* X, int count, float* Y, int accumulate,
         void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (type == Q3X_HIP_MATRIX_BF16) return Q3X_HIP_ENOTSUP;
    size_t bytes;
    if (!w || !X || !Y || count <= 0 || !quantized_size(type, rows, cols, &bytes))
        return Q3X_HIP_EINVAL;
    if (workspace_bytes > 0 && !workspace) return Q3X_HIP_EINVAL;
    const int bpr = cols / kBlock;
    const size_t row_bytes = static_cast<size_t>(bpr) * block_bytes(type);
    if (!aligned(w, 2) || !aligned(X, 16) || !aligned(Y, 4)) {
        // Unaligned operands: one matvec per token (the reference CPU prefill
        // is exactly this, engine.cpp:580-583).
        for (int t = 0; t < count; ++t) {
            const int status = q3x_hip_mv(w, type, rows, cols, X + static_cast<size_t>(t) * cols,
                                          Y + static_cast<size_t>(t) * rows, accumulate, stream);
            if (status != Q3X_HIP_OK) return status;
        }
        return Q3X_HIP_OK;
    }
    // The split plan runs only with all of the workspace it asks for (16-byte
    // aligned); otherwise q3x_hip_gemm's plan.
    const size_t need = x3_plan(rows, count, cols, false, SIZE_MAX).workspace_bytes();
    const size_t usable = need > 0 && aligned(workspace, 16) && workspace_bytes >= need ? need : 0;
    DenseGemm g{0, X, cols, count, static_cast<const uint8_t*>(w), row_bytes, Y, rows, accumulate != 0, 1,
                static_cast<float*>(workspace)};
    return type == Q3X_HIP_MATRIX_Q8_0 ? launch_x3<Q3X_HIP_MATRIX_Q8_0>(g, rows, count, cols, stream, usable)
                                       : launch_x3<Q3X_HIP_MATRIX_Q4_0>(g, rows, count, cols, stream, usable);
}

}  // namespace

extern "C" int q3x_hip_gemm(const void* w, uint32_t type, int rows, int cols, const float* X,
                            int count, float* Y, int accumulate, hipStream_t stream) {
    return gemm(w, type, rows, cols, X, count, Y, accumulate, nullptr, 0, stream);
}

extern "C" size_t q3x_hip_gemm_workspace_bytes(uint32_t type, int rows, int cols, int count) {
    size_t bytes;
    if (type == Q3X_HIP_MATRIX_BF16 || count <= 0 || !quantized_size(type, rows, cols, &bytes)) return 0;
    return x3_plan(rows, count, cols, false, SIZE_MAX).workspace_bytes();
}

extern "C" int q3x_hip_gemm_ws(const void* w, uint32_t type, int rows, int cols, const float* X, int count,
                               float* Y, int accumulate, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
    return gemm(w, type, rows, cols, X, count, Y, accumulate, workspace, workspace_bytes, stream);
}
