// matvec.hip -- q3x_hip_mv: the dense decode matvec entry point (kernels in
// matvec.h).
#include "matvec.h"

using namespace q3x;

extern "C" int q3x_hip_mv(const void* w, uint32_t type, int rows, int cols, const float* x,
                          float* y, int accumulate, hipStream_t stream) {
    if (type == Q3X_HIP_MATRIX_BF16) return Q3X_HIP_ENOTSUP;
    size_t bytes;
    if (!w || !x || !y || !quantized_size(type, rows, cols, &bytes)) return Q3X_HIP_EINVAL;
    const int bpr = cols / kBlock;
    const size_t row_bytes = static_cast<size_t>(bpr) * block_bytes(type);
    const bool staged = aligned(w, 16) && aligned(x, 16) && row_bytes % 16 == 0;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    if (accumulate) {
        const DenseRows<true> map{wb, row_bytes, x, y};
        return type == Q3X_HIP_MATRIX_Q8_0 ? launch_mv<Q3X_HIP_MATRIX_Q8_0>(map, rows, bpr, staged, stream)
                                           : launch_mv<Q3X_HIP_MATRIX_Q4_0>(map, rows, bpr, staged, stream);
    }
    const DenseRows<false> map{wb, row_bytes, x, y};
    return type == Q3X_HIP_MATRIX_Q8_0 ? launch_mv<Q3X_HIP_MATRIX_Q8_0>(map, rows, bpr, staged, stream)
                                       : launch_mv<Q3X_HIP_MATRIX_Q4_0>(map, rows, bpr, staged, stream);
}

extern "C" int q3x_hip_mv_multi(const q3x_hip_mv_item* items, int count, uint32_t type, int cols,
                                const float* x, hipStream_t stream) {
    if (type == Q3X_HIP_MATRIX_BF16) return Q3X_HIP_ENOTSUP;
    if (!items || !x || count < 1 || count > MultiRows::kMax || !is_quant_type(type) || cols <= 0 ||
        cols % kBlock != 0)
        return Q3X_HIP_EINVAL;
    const int bpr = cols / kBlock;
    const size_t row_bytes = static_cast<size_t>(bpr) * block_bytes(type);
    MultiRows map{};
    map.count = count;
    map.row_bytes = row_bytes;
    map.x = x;
    long long total = 0;
    bool staged = aligned(x, 16) && row_bytes % 16 == 0;
    for (int i = 0; i < count; ++i) {
        size_t bytes;
        const q3x_hip_mv_item& it = items[i];
        if (!it.weight || !it.out || !quantized_size(type, it.rows, cols, &bytes)) return Q3X_HIP_EINVAL;
        total += it.rows;
        if (total > INT32_MAX) return Q3X_HIP_EINVAL;
        map.w[i] = static_cast<const uint8_t*>(it.weight);
        map.y[i] = it.out;
        map.end[i] = static_cast<int>(total);
        if (it.accumulate) map.accumulate_mask |= 1u << i;
        staged = staged && aligned(it.weight, 16);
    }
    for (int i = count; i < MultiRows::kMax; ++i) {
        map.w[i] = map.w[0];
        map.y[i] = map.y[0];
        map.end[i] = static_cast<int>(total);
    }
    const int rows = static_cast<int>(total);
    int status = Q3X_HIP_ENOTSUP;
    if (staged)
        status = type == Q3X_HIP_MATRIX_Q8_0 ? launch_pipe_for<Q3X_HIP_MATRIX_Q8_0>(map, rows, bpr, stream)
                                             : launch_pipe_for<Q3X_HIP_MATRIX_Q4_0>(map, rows, bpr, stream);
    if (status != Q3X_HIP_ENOTSUP) return status;
    // Unaligned, or x too long for LDS: one launch per matrix.
    for (int i = 0; i < count; ++i) {
        status = q3x_hip_mv(items[i].weight, type, items[i].rows, cols, x, items[i].out, items[i].accumulate, stream);
        if (status != Q3X_HIP_OK) return status;
    }
    return Q3X_HIP_OK;
}
