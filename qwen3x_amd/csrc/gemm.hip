// gemm.hip -- q3x_hip_gemm: dense prefill GEMM Y[count, rows] (+)= X W^T
// with Q8_0 / Q4_0 weights on FP32 MFMA (kernel in gemm.h).
//
// Replaces the reference's batch_mv (arch/cuda/engine.cu:1568-1597), whose Q8
// path is an FP32 SIMT kernel (batch_mv_q8_kernel :761, 64 rows x 128 tokens
// per CTA) and which has no Q4_0 GEMM (it asserts, :1580).
#include "gemm.h"
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

// Tile shapes (WM x WN waves, each TM x TN tiles of 32x32): 128 x 128 on 8
// waves, 64 tokens x 128 weight rows on 8 waves, 64 x 64 on 4 waves.  A
// launch lasts about (tiles of the CU that takes the most, ceil(tiles /
// 256)) x (one tile's work, padded rows and tokens included) / (the shape's
// rate); the launch takes the shape with the least.  Rates measured on
// MI355X (TFLOP/s over full tiles): Q8_0 130 / 120 / 118, Q4_0 128 / 126 /
// 117.  E.g. 2048 tokens x 5120 rows: 640 tiles of 128 x 128 (3 on some CUs)
// against 1280 of 64 x 128 (5 each, half the work each): the latter, 126
// TFLOP/s against 104 measured; 48 rows: 32 tiles of 64 x 64.
template <uint32_t QT, int WM, int WN, int TM, int TN, int PF>
int launch_dense_gemm_tiles(const DenseGemm& base, hipStream_t stream) {
    constexpr int BM = WM * TM * 32, BN = WN * TN * 32;
    DenseGemm g = base;
    g.tiles_x = (base.rows + BN - 1) / BN;
    const long long tiles = static_cast<long long>(g.tiles_x) * ((base.count + BM - 1) / BM);
    if (tiles > 0x7fffffffLL) return Q3X_HIP_EINVAL;
    hipLaunchKernelGGL((gemm_mfma_kernel<QT, WM, WN, TM, TN, DenseGemm, PF>), dim3(static_cast<unsigned>(tiles)),
                       dim3(WM * WN * kWave), 0, stream, g, base.rows, base.cols);
    return launch_status();
}

// Register sets for the stages ahead (PF), measured per tile: two for Q8_0's
// 64 x 128 tiles, one elsewhere (equal or faster, fewer registers).
template <uint32_t QT>
int launch_dense_gemm(const DenseGemm& g, hipStream_t stream) {
    const bool q8 = QT == Q3X_HIP_MATRIX_Q8_0;
    auto cost = [&](int bm, int bn, double rate) {
        const long long tiles = static_cast<long long>((g.rows + bn - 1) / bn) * ((g.count + bm - 1) / bm);
        return static_cast<double>((tiles + kCUs - 1) / kCUs) * bm * bn / rate;
    };
    const double large = cost(128, 128, q8 ? 130.0 : 128.0);
    const double wide = cost(64, 128, q8 ? 120.0 : 126.0);
    const double small = cost(64, 64, q8 ? 118.0 : 117.0);
    if (large <= wide && large <= small) return launch_dense_gemm_tiles<QT, 2, 4, 2, 1, 1>(g, stream);
    if (wide <= small) {
        if (q8) return launch_dense_gemm_tiles<QT, 2, 4, 1, 1, 2>(g, stream);
        return launch_dense_gemm_tiles<QT, 2, 4, 1, 1, 1>(g, stream);
    }
    return launch_dense_gemm_tiles<QT, 2, 2, 1, 1, 1>(g, stream);
}

}  // namespace q3x

using namespace q3x;

extern "C" int q3x_hip_gemm(const void* w, uint32_t type, int rows, int cols, const float* X,
                            int count, float* Y, int accumulate, hipStream_t stream) {
    if (type == Q3X_HIP_MATRIX_BF16) return Q3X_HIP_ENOTSUP;
    size_t bytes;
    if (!w || !X || !Y || count <= 0 || !quantized_size(type, rows, cols, &bytes))
        return Q3X_HIP_EINVAL;
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
    DenseGemm g{0, X, cols, count, static_cast<const uint8_t*>(w), row_bytes, Y, rows, accumulate != 0};
    return type == Q3X_HIP_MATRIX_Q8_0 ? launch_dense_gemm<Q3X_HIP_MATRIX_Q8_0>(g, stream)
                                       : launch_dense_gemm<Q3X_HIP_MATRIX_Q4_0>(g, stream);
}
