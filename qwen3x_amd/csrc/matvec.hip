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
