// common.h -- block formats, argument checks and device helpers shared by the
// gfx950 kernels of the quantized-matmul backend.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "q3x_hip.h"

namespace q3x {

constexpr int kBlock = 32;        // weights per block (q8.h:8, q4.h:8)
constexpr int kQ8Bytes = 34;      // uint16 scale + int8[32]   (q8.h:10-15)
constexpr int kQ4Bytes = 18;      // uint16 scale + uint8[16]  (q4.h:12-15)
constexpr int kBF16Bytes = 64;    // 32 BF16 values (a block column of a BF16 matrix)
constexpr int kWave = 64;         // CDNA wavefront
constexpr int kCUs = 256;          // MI355X compute units

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Accesses of global memory through a pointer the compiler cannot trace to
// a kernel argument (a table entry picked at run time).  A plain access
// would be a flat instruction, which may address LDS as well as memory: the
// compiler then counts it in both wait counters and, with one in flight,
// waits for every outstanding load where it needs only the oldest (a
// prefetch ring then has nothing in flight across the loop's back edge).
__device__ __forceinline__ float load_global(const float* p) {
    typedef const __attribute__((address_space(1))) float GlobalFloat;
    return *(GlobalFloat*)p;
}
__device__ __forceinline__ void store_global(float* p, float v) {
    typedef __attribute__((address_space(1))) float GlobalFloat;
    *(GlobalFloat*)p = v;
}

__host__ __device__ constexpr int block_bytes(uint32_t type) {
    return type == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : kQ4Bytes;
}

// arch/cpu.cpp:161-179 with the same rejection rules.
inline bool quantized_size(uint32_t type, int rows, int cols, size_t* bytes) {
    size_t bb;
    if (type == Q3X_HIP_MATRIX_Q8_0) bb = kQ8Bytes;
    else if (type == Q3X_HIP_MATRIX_Q4_0) bb = kQ4Bytes;
    else return false;
    if (rows <= 0 || cols <= 0 || cols % kBlock != 0) return false;
    const size_t blocks = static_cast<size_t>(cols) / kBlock;
    const size_t maximum = SIZE_MAX;
    if (blocks > maximum / bb) return false;
    const size_t row_bytes = blocks * bb;
    if (static_cast<size_t>(rows) > maximum / row_bytes) return false;
    *bytes = static_cast<size_t>(rows) * row_bytes;
    return true;
}

inline bool is_quant_type(uint32_t type) {
    return type == Q3X_HIP_MATRIX_Q8_0 || type == Q3X_HIP_MATRIX_Q4_0;
}

inline bool aligned(const void* p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

// Launch-error check after an asynchronous kernel launch.
inline int launch_status() {
    return hipGetLastError() == hipSuccess ? Q3X_HIP_OK : Q3X_HIP_ERUNTIME;
}

// Exact IEEE binary16 -> binary32 by bit manipulation, identical bit for bit
// to the reference's f16() (arch/cpu.cpp:31-52), NaN payloads included.  Used
// where dequantised values are returned to the caller.
__device__ __forceinline__ float f16_exact(uint32_t value) {
    const uint32_t sign = (value & 0x8000u) << 16;
    const uint32_t exponent = (value >> 10) & 0x1fu;
    const uint32_t mantissa = value & 0x03ffu;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            // Normalise the subnormal: shift the leading one to bit 10.
            const int lead = __clz(mantissa) - 21;  // 1..10 shifts
            bits = sign | ((113u - lead) << 23) | (((mantissa << lead) & 0x03ffu) << 13);
        }
    } else if (exponent == 31) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    return __uint_as_float(bits);
}

// Hardware half -> float (v_cvt_f32_f16): exact for every finite value and
// infinity, subnormals included (f16 denormals are preserved on gfx950).
// Used inside the dot-product kernels.
__device__ __forceinline__ float f16_fast(uint32_t value) {
    _Float16 h;
    const uint16_t bits = static_cast<uint16_t>(value);
    __builtin_memcpy(&h, &bits, sizeof(h));
    return static_cast<float>(h);
}

// Signed byte k of a dword as float (one v_cvt_f32_i32_sdwa with sext).
template <int K>
__device__ __forceinline__ float sbyte(uint32_t v) {
    return static_cast<float>(static_cast<int8_t>(v >> (8 * K)));
}

// Lane exchange inside rows of 16 lanes through DPP (no LDS round trip).
// Controls (gfx9): quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E,
// row_half_mirror (lane i <- 7-i of its 8) = 0x141, row_mirror (i <- 15-i) =
// 0x140.  Every source lane lies inside the row, so no lane reads a bound.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}
__device__ __forceinline__ uint32_t read_lane_u32(uint32_t v, int lane) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}
__device__ __forceinline__ float read_lane_f32(float v, int lane) {
    return __uint_as_float(read_lane_u32(__float_as_uint(v), lane));
}

// Wave-wide maximum of an unsigned value, returned to every lane (uniform):
// xor-1, xor-2 and the two mirrors leave each row's maximum in all its lanes,
// then the four rows are compared.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0xB1>(v));
    v = max(v, dpp_u32<0x4E>(v));
    v = max(v, dpp_u32<0x141>(v));
    v = max(v, dpp_u32<0x140>(v));
    return max(max(read_lane_u32(v, 0), read_lane_u32(v, 16)), max(read_lane_u32(v, 32), read_lane_u32(v, 48)));
}
__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    return fmaxf(fmaxf(read_lane_f32(v, 0), read_lane_f32(v, 16)), fmaxf(read_lane_f32(v, 32), read_lane_f32(v, 48)));
}
// Wave-wide sum in a fixed tree order (pairs, quads, eights, rows, then
// (row0 + row1) + (row2 + row3)); every lane of a row sees the same bits at
// each level, because each level adds the same two values.
__device__ __forceinline__ float wave_sum_f32(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    return (read_lane_f32(v, 0) + read_lane_f32(v, 16)) + (read_lane_f32(v, 32) + read_lane_f32(v, 48));
}

// Sum over groups of WIDTH consecutive lanes (16, 32 or 64), returned to
// every lane of the group: DPP sums inside each row of 16 lanes (pairs,
// quads, eights, rows), then the row sums are added as scalars --
// (r0 + r1) for a 32-lane group, (r0 + r1) + (r2 + r3) for the wave.  A
// fixed order, so results are deterministic.  Call with every lane active.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(WIDTH == 16 || WIDTH == 32 || WIDTH == 64, "group of 16, 32 or 64 lanes");
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    if constexpr (WIDTH == 16) {
        return v;
    } else {
        const float r0 = read_lane_f32(v, 0), r1 = read_lane_f32(v, 16);
        const float r2 = read_lane_f32(v, 32), r3 = read_lane_f32(v, 48);
        if constexpr (WIDTH == 32) return (threadIdx.x & 32) ? r2 + r3 : r0 + r1;
        else return (r0 + r1) + (r2 + r3);
    }
}

// Orders LDS traffic of one wavefront: every lane's earlier LDS writes are
// visible to every lane's later LDS reads (LDS executes a wave's operations
// in issue order; this keeps the compiler from moving them across).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace q3x
