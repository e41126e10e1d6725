// matvec.h -- Q8_0 / Q4_0 dequant-dot matrix-vector products for decode
// (N = 1) on gfx950.
//
// Replaces the reference CUDA mv_q8_kernel / mv_add_q8_kernel / mv_q4_kernel /
// mv_add_q4_kernel (arch/cuda/engine.cu:546-612), which give one 256-thread
// block to each row and decode the fp16 scale per element.  Here:
//
//  * a wavefront owns G*RPI rows (G row groups of LPR lanes, RPI row
//    iterations); one lane owns one 32-weight block column of a pass, so its 32
//    activations stay in registers for all of the wave's rows;
//  * each pass stages the wave's row segments (LPR blocks per row) into the
//    wave's own LDS slice with coalesced 16-byte global loads.  Q8_0 rows of
//    8 blocks are 272 B = 17 x 16 B and Q4_0 rows 144 B = 9 x 16 B, so any
//    row whose length is a multiple of 256 columns starts 16-byte aligned;
//  * a lane reads its block back with aligned dword LDS reads and one
//    v_alignbyte per dword (blocks are 34 / 18 bytes, so they start on 2- or
//    4-byte boundaries), converts bytes with sign-extending SDWA converts and
//    accumulates in FP32 with FMAs: inner = sum q*x per block, then
//    acc += f16(d) * inner, the per-block factorisation of arch/cpu.cpp:64-73;
//  * Q4_0 nibbles become signed bytes 16*(n-8) with two logic ops per four
//    bytes (xor 0x88, mask / shift), so each weight costs one convert and one
//    FMA; the factor 16 is removed exactly by scaling d by 1/16;
//  * the row's lane partial sums are combined with a butterfly inside the
//    row group; lane 0 of the group writes (or adds to) y.
// Reduction order is fixed per shape, so results are deterministic.
#pragma once

#include "common.h"
#include "rows.h"

namespace q3x {

constexpr int kMvWaves = 4;  // wavefronts per workgroup

// Dot product of one Q8_0 block held in LDS (byte offset p) with x[0..31].
__device__ __forceinline__ float block_dot_q8(const uint8_t* lds, uint32_t p, const float* xv) {
    const uint32_t scale = *reinterpret_cast<const uint16_t*>(lds + p);
    const uint32_t start = p + 2;
    const uint32_t base = start & ~3u;
    const uint32_t shift = start & 3u;
    uint32_t a[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) a[k] = *reinterpret_cast<const uint32_t*>(lds + base + 4 * k);
    float even = 0.0f, odd = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
        const uint32_t q0 = __builtin_amdgcn_alignbyte(a[k + 1], a[k], shift);
        const uint32_t q1 = __builtin_amdgcn_alignbyte(a[k + 2], a[k + 1], shift);
        even = fmaf(sbyte<0>(q0), xv[4 * k + 0], even);
        odd = fmaf(sbyte<0>(q1), xv[4 * k + 4], odd);
        even = fmaf(sbyte<1>(q0), xv[4 * k + 1], even);
        odd = fmaf(sbyte<1>(q1), xv[4 * k + 5], odd);
        even = fmaf(sbyte<2>(q0), xv[4 * k + 2], even);
        odd = fmaf(sbyte<2>(q1), xv[4 * k + 6], odd);
        even = fmaf(sbyte<3>(q0), xv[4 * k + 3], even);
        odd = fmaf(sbyte<3>(q1), xv[4 * k + 7], odd);
    }
    return f16_fast(scale) * (even + odd);
}

// Dot product of one Q4_0 block held in LDS with x[0..31], returned as
// f16(d) * sum (n - 8) x.  Nibble bytes become signed 16*(n-8) bytes.
__device__ __forceinline__ float block_dot_q4(const uint8_t* lds, uint32_t p, const float* xv) {
    const uint32_t scale = *reinterpret_cast<const uint16_t*>(lds + p);
    const uint32_t start = p + 2;
    const uint32_t base = start & ~3u;
    const uint32_t shift = start & 3u;
    uint32_t a[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) a[k] = *reinterpret_cast<const uint32_t*>(lds + base + 4 * k);
    float lo_sum = 0.0f, hi_sum = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t u = __builtin_amdgcn_alignbyte(a[k + 1], a[k], shift) ^ 0x88888888u;
        const uint32_t hi = u & 0xF0F0F0F0u;         // 16*(high nibble - 8): elements 16+4k+j
        const uint32_t lo = (u << 4) & 0xF0F0F0F0u;  // 16*(low nibble - 8):  elements 4k+j
        lo_sum = fmaf(sbyte<0>(lo), xv[4 * k + 0], lo_sum);
        hi_sum = fmaf(sbyte<0>(hi), xv[16 + 4 * k + 0], hi_sum);
        lo_sum = fmaf(sbyte<1>(lo), xv[4 * k + 1], lo_sum);
        hi_sum = fmaf(sbyte<1>(hi), xv[16 + 4 * k + 1], hi_sum);
        lo_sum = fmaf(sbyte<2>(lo), xv[4 * k + 2], lo_sum);
        hi_sum = fmaf(sbyte<2>(hi), xv[16 + 4 * k + 2], hi_sum);
        lo_sum = fmaf(sbyte<3>(lo), xv[4 * k + 3], lo_sum);
        hi_sum = fmaf(sbyte<3>(hi), xv[16 + 4 * k + 3], hi_sum);
    }
    return (f16_fast(scale) * 0.0625f) * (lo_sum + hi_sum);
}

// Streaming kernel.  QT: matrix type; LPR: lanes (= block columns) per row
// group, 16/32/64; R: row iterations per batch.  A unit of work is a batch
// of RW = G*R rows (G = 64/LPR row groups) times one K pass of LPR blocks;
// lane li of row group g owns block column b0 + li of the pass, so its 32
// activations serve all R rows.  The grid is persistent (sized to what is
// resident at once, GW wavefronts) and each wave accumulates a batch's rows
// over all passes before storing them.
//
// Rows and activations: with XL every row reads the same x, which the
// workgroup copies once into LDS (padded 16 bytes per two blocks, so the 64
// lanes' 16-byte reads of consecutive blocks hit distinct banks), and wave
// gw takes the strided rows gw, gw + GW, gw + 2*GW, ...: every wave streams
// the same number of rows (+-1) whatever the row count, and at any moment
// the GPU reads one band of consecutive rows.  Without XL (inputs that change
// between groups of rows, e.g. per expert slot) a batch is RW consecutive
// rows and each unit reads its x slice from global memory.
//
// Weights: each row segment of a unit (LPR blocks = SEG bytes) is copied
// global -> LDS by direct-to-LDS buffer loads (non-temporal: weights are used
// once): SEG / 1 KB loads of 16 bytes per lane, then 256-byte loads of 4
// bytes per lane for the rest.  The buffer descriptor's range is the
// segment's bytes, so lanes past the end of a short segment, rows past the
// matrix and rows of an out-of-range expert read zeros; segments sit SEGP
// (SEG rounded up to 256) bytes apart in LDS so no lane writes into the next
// one.  The wave waits for its loads, then reads its blocks back with aligned
// dword reads (block_dot_q8 / block_dot_q4).  Latency is hidden by the other
// resident wavefronts.
// Requires: every row start 16-byte aligned, bpr % 8 == 0, bpr <= LPR when
// LPR < 64, x 16-byte aligned; rows of a batch read one input.
constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9)
constexpr int kNonTemporal = 2;           // buffer "nt" cache policy

template <uint32_t QT, int LPR, int R>
struct StagedShape {
    static constexpr int BB = QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : kQ4Bytes;
    static constexpr int G = kWave / LPR;
    static constexpr int RW = G * R;                      // rows per batch
    static constexpr int SEG = LPR * BB;                  // bytes of a full row segment
    static constexpr int J16 = SEG / 1024;                // 1 KB loads (16 B per lane)
    static constexpr int J4 = (SEG - 1024 * J16 + 255) / 256;  // 256 B loads (4 B per lane)
    static constexpr int SEGP = 1024 * J16 + 256 * J4;    // LDS pitch of a segment
    static constexpr int WAVE_LDS = RW * SEGP;            // LDS bytes per wave
};

// LDS offset of x block b in the padded layout: 16 spare bytes after every
// two 128-byte blocks, so blocks b..b+15 start in 16 distinct bank groups.
__host__ __device__ constexpr uint32_t x_block_offset(int b) { return 128u * b + 16u * (b >> 1); }
__host__ __device__ constexpr uint32_t x_lds_bytes(int bpr) { return x_block_offset(bpr) + 16u; }

template <uint32_t QT, int LPR, int R, bool XL, class Rows>
__global__ __launch_bounds__(512) void mv_stream_kernel(Rows rows, int nrows, int bpr) {
    using S = StagedShape<QT, LPR, R>;
    constexpr int BB = S::BB, G = S::G, RW = S::RW, J16 = S::J16, J4 = S::J4, SEGP = S::SEGP;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_dyn[];

    const int lane = threadIdx.x & (kWave - 1);
    // Wave-uniform (scalar) so that row pointers, buffer descriptors and LDS
    // bases live in SGPRs.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int wpb = blockDim.x / kWave;
    const int gw = blockIdx.x * wpb + wave;
    const int GW = gridDim.x * wpb;
    const int g = lane / LPR;
    const int li = lane % LPR;
    const uint32_t xbytes = XL ? x_lds_bytes(bpr) : 0u;
    uint8_t* const xl = lds_dyn;
    uint8_t* const wl = lds_dyn + ((xbytes + 15u) & ~15u) + wave * S::WAVE_LDS;
    const int npass = (bpr + LPR - 1) / LPR;
    // Batches of this wave: strided rows (XL) or consecutive row tiles.
    const int my_rows = XL ? (gw < nrows ? (nrows - gw + GW - 1) / GW : 0) : 0;
    const int batches = XL ? (my_rows + RW - 1) / RW : 0;
    const int tiles = (nrows + RW - 1) / RW;
    auto row_of = [&](int batch, int seg) {
        return XL ? gw + (batch * RW + seg) * GW : batch * RW + seg;
    };

    if (XL) {
        // x into LDS once: 16-byte chunk c of block b lands at
        // x_block_offset(b) + 16 * (c % 8).
        const f32x4* xs = reinterpret_cast<const f32x4*>(rows.input(0));
        for (int c = threadIdx.x; c < bpr * 8; c += blockDim.x)
            *reinterpret_cast<f32x4*>(xl + x_block_offset(c >> 3) + 16 * (c & 7)) = xs[c];
        __syncthreads();
    }

    // XL: batch index 0..batches-1 of this wave; otherwise tile index.
    for (int b = XL ? 0 : gw; XL ? b < batches : b < tiles; b += XL ? 1 : GW) {
        float acc[R];
#pragma unroll
        for (int it = 0; it < R; ++it) acc[it] = 0.0f;
        for (int pass = 0; pass < npass; ++pass) {
            const int b0 = pass * LPR;
            const int nb = min(LPR, bpr - b0);
#pragma unroll
            for (int seg = 0; seg < RW; ++seg) {
                const int row = row_of(b, seg);
                const uint8_t* src = row < nrows ? rows.row(row) : nullptr;
                const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<uint8_t*>(src ? src + static_cast<size_t>(b0) * BB : rows.any()), 0,
                    src ? nb * BB : 0, kBufferFlags);
                uint8_t* dst = wl + seg * SEGP;
#pragma unroll
                for (int j = 0; j < J16; ++j)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        rsrc, (__attribute__((address_space(3))) void*)(dst + j * 1024), 16, 16 * lane,
                        j * 1024, 0, kNonTemporal);
#pragma unroll
                for (int j = 0; j < J4; ++j)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        rsrc, (__attribute__((address_space(3))) void*)(dst + J16 * 1024 + j * 256), 4, 4 * lane,
                        J16 * 1024 + j * 256, 0, kNonTemporal);
            }
            float xv[32];
            const int col = li < nb ? b0 + li : 0;  // lanes past the pass read block 0 (unused)
            if (XL) {
                const uint8_t* xs = xl + x_block_offset(col);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const f32x4 t = *reinterpret_cast<const f32x4*>(xs + 16 * i);
                    xv[4 * i + 0] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w;
                }
            } else {
                const f32x4* xs = reinterpret_cast<const f32x4*>(
                    rows.input(min(row_of(b, g), nrows - 1)) + 32 * col);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const f32x4 t = xs[i];
                    xv[4 * i + 0] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w;
                }
            }
            // The direct-to-LDS loads (and any x loads) have landed.
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            wave_lds_sync();
            if (li < nb) {
#pragma unroll
                for (int it = 0; it < R; ++it) {
                    const uint32_t p = (it * G + g) * SEGP + li * BB;
                    acc[it] += QT == Q3X_HIP_MATRIX_Q8_0 ? block_dot_q8(wl, p, xv) : block_dot_q4(wl, p, xv);
                }
            }
            // Every lane's LDS reads are consumed before the next unit refills.
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            wave_lds_sync();
        }
#pragma unroll
        for (int it = 0; it < R; ++it) {
            const float total = group_sum<LPR>(acc[it]);
            const int row = row_of(b, it * G + g);
            if (li == 0 && row < nrows) rows.store(row, rows.previous(row) + total);
        }
    }
}

// Any alignment, any cols % 32 == 0: one wave per row, byte loads.  Used for
// shapes the staged kernel does not take (e.g. rows that are not a multiple
// of 256 columns long, or unaligned pointers).
template <uint32_t QT, class Rows>
__global__ __launch_bounds__(kMvWaves * kWave) void mv_generic_kernel(Rows rows, int nrows, int bpr) {
    constexpr int BB = QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : kQ4Bytes;
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kMvWaves + threadIdx.x / kWave;
    if (row >= nrows) return;
    const uint8_t* src = rows.row(row);
    const float* x = rows.input(row);
    float acc = 0.0f;
    if (src) {
        for (int b = lane; b < bpr; b += kWave) {
            const uint8_t* blk = src + static_cast<size_t>(b) * BB;
            const float scale = f16_fast(blk[0] | (blk[1] << 8));
            const float* xb = x + 32 * b;
            float inner = 0.0f;
            if (QT == Q3X_HIP_MATRIX_Q8_0) {
                for (int i = 0; i < 32; ++i)
                    inner = fmaf(static_cast<float>(static_cast<int8_t>(blk[2 + i])), xb[i], inner);
            } else {
                for (int i = 0; i < 16; ++i) {
                    const uint32_t packed = blk[2 + i];
                    inner = fmaf(static_cast<float>(static_cast<int>(packed & 15u) - 8), xb[i], inner);
                }
                for (int i = 0; i < 16; ++i) {
                    const uint32_t packed = blk[2 + i];
                    inner = fmaf(static_cast<float>(static_cast<int>(packed >> 4) - 8), xb[16 + i], inner);
                }
            }
            acc = fmaf(scale, inner, acc);
        }
    }
    const float total = group_sum<kWave>(acc);
    if (lane == 0) rows.store(row, rows.previous(row) + total);
}

// ---- launch helpers shared with the MoE decode path ----

// Persistent grid sized to what is resident at once on 256 CUs: workgroups
// of 4 (or 8) wavefronts, as many per CU as LDS allows (at most 2 of 4 or 1
// of 8 = 8 wavefronts per CU, the occupancy that streams best), never more
// workgroups than row tiles need.
constexpr int kCUs = 256;
constexpr size_t kLdsPerCU = 160 * 1024;

template <uint32_t QT, int LPR, int R, bool XL, class Rows>
inline int launch_stream(const Rows& rows, int nrows, int bpr, int wpb, size_t lds, int wgs_per_cu,
                         hipStream_t stream) {
    using S = StagedShape<QT, LPR, R>;
    auto kernel = mv_stream_kernel<QT, LPR, R, XL, Rows>;
    // Allow the largest dynamic LDS this instantiation can use (once per
    // process: the first call of each instantiation, typically eager).
    static const bool lds_ready =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(kLdsPerCU)) == hipSuccess;
    if (lds > 64 * 1024 && !lds_ready) return Q3X_HIP_ERUNTIME;
    // XL: at most one wavefront per row; otherwise one per row tile.
    const long long units = XL ? nrows : (nrows + S::RW - 1) / S::RW;
    const long long need = (units + wpb - 1) / wpb;
    const int grid = static_cast<int>(std::min<long long>(need, static_cast<long long>(kCUs) * wgs_per_cu));
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kWave * wpb), lds, stream, rows, nrows, bpr);
    return launch_status();
}

// Launch plan for one R: workgroup size, workgroups per CU, LDS bytes.
struct StreamPlan {
    int wpb = 0, per_cu = 0;
    size_t lds = 0;
    bool ok = false;
};

inline StreamPlan plan_stream(size_t xb, int wave_lds) {
    StreamPlan p;
    // 8 resident wavefronts per CU: one workgroup of 8 (measured slightly
    // ahead), else two of 4.
    if (xb + 8u * wave_lds <= kLdsPerCU) { p.wpb = 8; p.per_cu = 1; p.lds = xb + 8u * wave_lds; p.ok = true; }
    else if ((xb + 4u * wave_lds) * 2 <= kLdsPerCU) { p.wpb = 4; p.per_cu = 2; p.lds = xb + 4u * wave_lds; p.ok = true; }
    return p;
}

// Chooses R for LPR lanes per row.  XL (strided rows): batch sizes measured
// best per shape class (below).  Otherwise (consecutive tiles), the cost of a candidate is the
// rows one wavefront streams -- ceil(tiles / waves) * rows per tile, so
// uneven tile counts are charged -- times the extra x traffic of small tiles.
template <uint32_t QT, int LPR, bool XL, class Rows>
inline int launch_staged(const Rows& rows, int nrows, int bpr, hipStream_t stream) {
    const size_t xb = XL ? ((x_lds_bytes(bpr) + 15) & ~size_t{15}) : 0;
    const StreamPlan p4 = plan_stream(xb, StagedShape<QT, LPR, 4>::WAVE_LDS);
    const StreamPlan p2 = plan_stream(xb, StagedShape<QT, LPR, 2>::WAVE_LDS);
    const StreamPlan p1 = plan_stream(xb, StagedShape<QT, LPR, 1>::WAVE_LDS);
    const bool q8 = QT == Q3X_HIP_MATRIX_Q8_0;
    if (XL) {
        // Q8_0: 4-row batches once every wavefront has many rows (lm_head),
        // 2-row batches for matrices of a few rows per wavefront; Q4_0: 4.
        const long long waves = static_cast<long long>(kCUs) * 8;
        const int target = !q8 ? 4 : (nrows >= 16 * waves ? 4 : (nrows >= waves ? 2 : 1));
        if (target >= 4 && p4.ok)
            return launch_stream<QT, LPR, 4, XL>(rows, nrows, bpr, p4.wpb, p4.lds, p4.per_cu, stream);
        if (target >= 2 && p2.ok)
            return launch_stream<QT, LPR, 2, XL>(rows, nrows, bpr, p2.wpb, p2.lds, p2.per_cu, stream);
        if (p1.ok) return launch_stream<QT, LPR, 1, XL>(rows, nrows, bpr, p1.wpb, p1.lds, p1.per_cu, stream);
        return Q3X_HIP_ENOTSUP;  // x too long for LDS: caller uses the global-x variant
    }
    auto cost = [&](const StreamPlan& p, int r, double x_factor) {
        if (!p.ok) return 1e300;
        const long long rw = static_cast<long long>(kWave / LPR) * r;
        const long long tiles = (nrows + rw - 1) / rw;
        const long long waves = static_cast<long long>(kCUs) * p.per_cu * p.wpb;
        return static_cast<double>((tiles + waves - 1) / waves) * rw * x_factor;
    };
    const double c4 = cost(p4, 4, 1.0);
    const double c2 = cost(p2, 2, q8 ? 1.15 : 1.3);
    const double c1 = cost(p1, 1, q8 ? 1.5 : 2.0);
    if (c4 <= c2 && c4 <= c1 && p4.ok)
        return launch_stream<QT, LPR, 4, XL>(rows, nrows, bpr, p4.wpb, p4.lds, p4.per_cu, stream);
    if (c2 <= c1 && p2.ok)
        return launch_stream<QT, LPR, 2, XL>(rows, nrows, bpr, p2.wpb, p2.lds, p2.per_cu, stream);
    return launch_stream<QT, LPR, 1, XL>(rows, nrows, bpr, p1.wpb, p1.lds, p1.per_cu, stream);
}

template <uint32_t QT, class Rows>
int launch_mv(const Rows& rows, int nrows, int bpr, bool staged, hipStream_t stream) {
    if (!staged) {
        const int grid = (nrows + kMvWaves - 1) / kMvWaves;
        hipLaunchKernelGGL((mv_generic_kernel<QT, Rows>), dim3(grid), dim3(kMvWaves * kWave), 0,
                           stream, rows, nrows, bpr);
        return launch_status();
    }
    // x shared by all rows (and short enough for LDS): staged once per
    // workgroup; otherwise per unit from global memory.
    int status = Q3X_HIP_ENOTSUP;
    if (bpr <= 16) {
        if constexpr (Rows::kSharedInput) status = launch_staged<QT, 16, true>(rows, nrows, bpr, stream);
        if (status == Q3X_HIP_ENOTSUP) status = launch_staged<QT, 16, false>(rows, nrows, bpr, stream);
    } else if (bpr <= 32) {
        if constexpr (Rows::kSharedInput) status = launch_staged<QT, 32, true>(rows, nrows, bpr, stream);
        if (status == Q3X_HIP_ENOTSUP) status = launch_staged<QT, 32, false>(rows, nrows, bpr, stream);
    } else {
        if constexpr (Rows::kSharedInput) status = launch_staged<QT, 64, true>(rows, nrows, bpr, stream);
        if (status == Q3X_HIP_ENOTSUP) status = launch_staged<QT, 64, false>(rows, nrows, bpr, stream);
    }
    return status;
}

}  // namespace q3x

