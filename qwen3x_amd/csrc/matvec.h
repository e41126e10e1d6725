// matvec.h -- Q8_0 / Q4_0 dequant-dot matrix-vector products for decode
// (N = 1) on gfx950.
//
// Replaces the reference CUDA mv_q8_kernel / mv_add_q8_kernel / mv_q4_kernel /
// mv_add_q4_kernel (arch/cuda/engine.cu:546-612), which give one 256-thread
// block to each row and decode the fp16 scale per element.  Here:
//
//  * one lane owns one 32-weight block column of a pass of LPR blocks, so its
//    32 activations stay in registers for all the rows the wave streams;
//  * row segments arrive with coalesced 16-byte buffer loads and go through
//    the wave's LDS slice, where each lane reads its own block back with
//    aligned dword reads and one v_alignbyte per dword (blocks are 34 / 18
//    bytes, so they start on 2- or 4-byte boundaries).  Q8_0 rows of 8 blocks
//    are 272 B = 17 x 16 B and Q4_0 rows 144 B = 9 x 16 B, so any row whose
//    length is a multiple of 256 columns starts 16-byte aligned;
//  * Q8_0 bytes convert with sign-extending SDWA converts and accumulate in
//    FP32 with FMAs: inner = sum q*x per block, then acc += f16(d) * inner,
//    the per-block factorisation of arch/cpu.cpp:64-73;
//  * Q4_0 nibbles become the exact binary16 values n - 8 that v_fma_mix_f32
//    takes directly (block_dot_q4_exact), or signed bytes 16*(n-8) for the
//    SDWA path (block_dot_q4);
//  * the row's lane partial sums are combined with a butterfly inside the
//    row group; lane 0 of the group writes (or adds to) y.
// mv_pipe_kernel (x shared by all rows, held in LDS) prefetches the next
// step's weights into registers while the current step computes;
// mv_stream_kernel (x per row group, e.g. per expert slot) stages weights
// with direct-to-LDS loads.  Reduction order is fixed per shape, so results
// are deterministic.
#pragma once

#include <type_traits>

#include "common.h"
#include "rows.h"

namespace q3x {

// Row maps that choose their rows inside the launch (kRouteLds: the LDS
// bytes their route() needs after the waves' slices): route() runs first,
// with every thread of the workgroup, and returns what for_wave reads.
template <class R, class = void>
struct rows_route {
    static constexpr bool value = false;
    static constexpr uint32_t lds = 0;
};
template <class R>
struct rows_route<R, std::void_t<decltype(R::kRouteLds)>> {
    static constexpr bool value = true;
    static constexpr uint32_t lds = R::kRouteLds;
};

// A wave's rows: for_wave, after route() for row maps that route.
template <class Rows, bool = rows_route<Rows>::value>
struct WaveRows {
    __device__ static auto get(const Rows& r, int& gw, int& GW, int& nrows, uint8_t*) { return r.for_wave(gw, GW, nrows); }
};
template <class Rows>
struct WaveRows<Rows, true> {
    __device__ static auto get(const Rows& r, int& gw, int& GW, int& nrows, uint8_t* lds) {
        return r.for_wave(gw, GW, nrows, r.route(lds));
    }
};

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

constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9)
constexpr int kNonTemporal = 2;           // buffer "nt" cache policy

// LDS offset of x block b in the padded layout: 16 spare bytes after every
// two 128-byte blocks, so the 16-byte reads of 16 consecutive blocks start in
// 16 distinct bank groups.
__host__ __device__ constexpr uint32_t x_block_offset(int b) { return 128u * b + 16u * (b >> 1); }
__host__ __device__ constexpr uint32_t x_lds_bytes(int bpr) { return x_block_offset(bpr) + 16u; }

// Streaming kernel for rows whose input changes between row groups (the
// down projections of routed experts, one input per slot), and for inputs
// too long for LDS.  QT: matrix type; LPR: lanes (= block columns) per row
// group, 16/32/64; R: row iterations per batch.  A unit of work is a tile of
// RW = G*R consecutive rows (G = 64/LPR row groups) times one K pass of LPR
// blocks; lane li of row group g owns block column b0 + li of the pass and
// reads its 32 activations from global memory, so they serve all R rows.
// The grid is persistent (sized to what is resident at once, GW wavefronts,
// which take tiles round-robin); a wave accumulates a tile over all passes
// before storing it.
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
// Requires: every row start 16-byte aligned, bpr % 8 == 0, x 16-byte aligned;
// the rows of a tile read one input.
template <uint32_t QT, int LPR, int R>
struct StagedShape {
    static constexpr int BB = QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : kQ4Bytes;
    static constexpr int G = kWave / LPR;
    static constexpr int RW = G * R;                      // rows per tile
    static constexpr int SEG = LPR * BB;                  // bytes of a full row segment
    static constexpr int J16 = SEG / 1024;                // 1 KB loads (16 B per lane)
    static constexpr int J4 = (SEG - 1024 * J16 + 255) / 256;  // 256 B loads (4 B per lane)
    static constexpr int SEGP = 1024 * J16 + 256 * J4;    // LDS pitch of a segment
    static constexpr int WAVE_LDS = RW * SEGP;            // LDS bytes per wave
};

template <uint32_t QT, int LPR, int R, class Rows>
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
    uint8_t* const wl = lds_dyn + wave * S::WAVE_LDS;
    const int npass = (bpr + LPR - 1) / LPR;
    const int tiles = (nrows + RW - 1) / RW;

    for (int b = gw; b < tiles; b += GW) {
        float acc[R];
#pragma unroll
        for (int it = 0; it < R; ++it) acc[it] = 0.0f;
        for (int pass = 0; pass < npass; ++pass) {
            const int b0 = pass * LPR;
            const int nb = min(LPR, bpr - b0);
#pragma unroll
            for (int seg = 0; seg < RW; ++seg) {
                const int row = b * RW + seg;
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
            {
                const f32x4* xs = reinterpret_cast<const f32x4*>(rows.input(min(b * RW + g, nrows - 1)) + 32 * col);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const f32x4 t = xs[i];
                    xv[4 * i + 0] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w;
                }
            }
            // The direct-to-LDS loads (and the x loads) have landed.
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
            const int row = b * RW + it * G + g;
            if (li == 0 && row < nrows) rows.store(row, rows.previous(row) + total);
        }
    }
}

// Q4_0 block dot with every weight exact in binary16.  A nibble n placed in
// bits 0-3 of a half whose other bits are 0x6400 is the half 1024 + n
// (exponent 2^10, n in the last mantissa bits); placed in bits 4-7 it is
// 1024 + 16n.  One v_and_or per half pair builds those, one packed half add
// of -1032 (-1152) turns them into n - 8 (16 (n - 8)) exactly, and
// v_fma_mix_f32 multiplies such a half by an FP32 activation exactly.  So
// the block's inner product is the reference's sum of (n - 8) x
// (arch/cpu.cpp:91-101) with exact products and FP32 sums: elements 0..15
// and 16..31 in two chains (the second 16 times its value), joined by one
// FMA with 1/16.  Its rounding is relative to sum |n - 8| |x|, as the
// reference's is, and a block of zero weights (all nibbles 8) gives 0.
// Returns f16(d) times that.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_half2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }

// (a & mask) | bits in one v_and_or_b32.  A VOP3 instruction on gfx9 takes
// no literal and one scalar operand, so the compiler would split it into an
// AND and an OR with literals; the mask rides in a VGPR, the bits in an SGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(mask), "s"(bits));
    return r;
}

__device__ __forceinline__ float block_dot_q4_exact(const uint8_t* lds, uint32_t p, const float* xv) {
    const uint32_t scale = *reinterpret_cast<const uint16_t*>(lds + p);
    const uint32_t start = p + 2;
    const uint32_t base = start & ~3u;
    const uint32_t shift = start & 3u;
    uint32_t a[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) a[k] = *reinterpret_cast<const uint32_t*>(lds + base + 4 * k);
    const half2_t lo_bias = as_half2(0xE408E408u);  // -1032: 1024 + n -> n - 8
    const half2_t hi_bias = as_half2(0xE480E480u);  // -1152: 1024 + 16n -> 16 (n - 8)
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        // Bytes 4k..4k+3: low nibble of byte j is element j, high nibble 16 + j.
        const uint32_t u = __builtin_amdgcn_alignbyte(a[k + 1], a[k], shift);
        const uint32_t t = u >> 8;
        const half2_t e0 = as_half2(and_or(u, 0x000F000Fu, 0x64006400u)) + lo_bias;  // elements 4k, 4k+2
        const half2_t e1 = as_half2(and_or(u, 0x00F000F0u, 0x64006400u)) + hi_bias;  // 16+4k, 16+4k+2 (x16)
        const half2_t e2 = as_half2(and_or(t, 0x000F000Fu, 0x64006400u)) + lo_bias;  // 4k+1, 4k+3
        const half2_t e3 = as_half2(and_or(t, 0x00F000F0u, 0x64006400u)) + hi_bias;  // 16+4k+1, 16+4k+3 (x16)
        lo = fmaf(static_cast<float>(e0.x), xv[4 * k + 0], lo);
        hi = fmaf(static_cast<float>(e1.x), xv[16 + 4 * k + 0], hi);
        lo = fmaf(static_cast<float>(e2.x), xv[4 * k + 1], lo);
        hi = fmaf(static_cast<float>(e3.x), xv[16 + 4 * k + 1], hi);
        lo = fmaf(static_cast<float>(e0.y), xv[4 * k + 2], lo);
        hi = fmaf(static_cast<float>(e1.y), xv[16 + 4 * k + 2], hi);
        lo = fmaf(static_cast<float>(e2.y), xv[4 * k + 3], lo);
        hi = fmaf(static_cast<float>(e3.y), xv[16 + 4 * k + 3], hi);
    }
    return f16_fast(scale) * fmaf(hi, 0.0625f, lo);
}

// Software-pipelined streaming kernel for inputs shared by every row (x held
// in LDS, once per workgroup).  D: steps in flight per wave (a ring of
// register buffers); WPE: minimum waves per SIMD the build must allow (8
// caps it at 64 VGPRs).  A wave works on G = 64 / LPR rows at a time,
// LPR lanes per row, one lane per 32-weight block column of an LPR-block
// pass; it owns the strided rows gw, gw + GW, ... in batches of G * R.  A
// step is one (batch, pass): its G * R row segments arrive in registers by
// 16-byte buffer loads issued D steps ahead, so the loads of steps s+1..s+D
// are in flight while step s computes.  The G segments of a row iteration are
// written to the wave's LDS slice (reused iteration after iteration: LDS
// executes a wave's operations in issue order) and read back block-wise.
// Rows past the matrix, and the prefetch after the last step, use an empty
// buffer range, which reads zeros without touching memory.
// Requires: rows 16-byte aligned, bpr % 8 == 0, x 16-byte aligned.
template <uint32_t QT, int LPR>
struct PipeShape {
    static constexpr int BB = QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : kQ4Bytes;
    static constexpr int G = kWave / LPR;           // rows in flight per wave
    static constexpr int SEG = LPR * BB;            // bytes of a full row segment
    static constexpr int J = (SEG + 1023) / 1024;   // 16-byte loads per lane per segment
    static constexpr int SEGP = 1024 * J;           // LDS bytes per segment
    static constexpr int WAVE_LDS = G * SEGP;       // LDS bytes per wave
};

// LDS bytes of the shared part of a pipe launch: x (padded).
__host__ __device__ constexpr uint32_t pipe_x_bytes(int bpr) { return (x_lds_bytes(bpr) + 15u) & ~15u; }

// Input staging of mv_pipe_kernel: the launch's x (bpr blocks of 32 FP32
// values) into the workgroup's padded LDS copy, once per workgroup, with
// every thread of the workgroup taking part.  Other stagings (a norm or an
// activation applied on the way in) supply the same stage() member; `work`
// is 1 KB of LDS that is free until the staging's last barrier.
struct PlainInput {
    __device__ void stage(const float* x, uint8_t* xl, int bpr, float* /*work*/) const {
        const f32x4* xs = reinterpret_cast<const f32x4*>(x);
        for (int c = threadIdx.x; c < bpr * 8; c += blockDim.x)
            *reinterpret_cast<f32x4*>(xl + x_block_offset(c >> 3) + 16 * (c & 7)) = xs[c];
        __syncthreads();
    }
};

template <uint32_t QT, int LPR, int R, int D, class Rows, int WPE, class In = PlainInput>
__global__ __launch_bounds__(1024, WPE) void mv_pipe_kernel(Rows all_rows, int nrows, int bpr, In in) {
    using S = PipeShape<QT, LPR>;
    constexpr int BB = S::BB, G = S::G, J = S::J, RS = G * R;
    constexpr bool Q4 = QT == Q3X_HIP_MATRIX_Q4_0;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_dyn[];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int wpb = blockDim.x / kWave;
    int gw = blockIdx.x * wpb + wave;
    int GW = gridDim.x * wpb;
    // The wave's matrix (multi-matrix launches); gw, GW, nrows become its own.
    const auto rows = WaveRows<Rows>::get(all_rows, gw, GW, nrows, lds_dyn + pipe_x_bytes(bpr) + wpb * S::WAVE_LDS);
    const int g = lane / LPR;
    const int li = lane % LPR;
    uint8_t* const xl = lds_dyn;
    uint8_t* const wl = lds_dyn + pipe_x_bytes(bpr) + wave * S::WAVE_LDS;
    const int npass = (bpr + LPR - 1) / LPR;
    const int my_rows = gw < nrows ? (nrows - gw + GW - 1) / GW : 0;
    const int steps = (my_rows + RS - 1) / RS * npass;

    // Ring of D steps in flight: step s lives in pre[s % D].
    u32x4 pre[D][RS][J];
    // Row starts of the batch being requested, found once per batch (the
    // passes of a batch only add their offset); null for rows past the
    // matrix -- every row of a batch past the wave's last -- and rows of an
    // expert id out of range.
    const uint8_t* qrow[RS];
    auto find_rows = [&](int b) {
#pragma unroll
        for (int i = 0; i < RS; ++i) {
            const int row = gw + (b * RS + i) * GW;
            qrow[i] = row < nrows ? rows.row(row) : nullptr;
        }
    };
    // Loads of row i of the requested batch's pass p into pre[d][i]; a null
    // row gives zeros.
    auto issue_row = [&](int d, int p, int i) {
        const int b0 = p * LPR;
        const uint8_t* base = qrow[i];
        const uint8_t* src = base ? base + static_cast<size_t>(b0) * BB : rows.any();
        const int bytes = base ? min(LPR, bpr - b0) * BB : 0;
        const __amdgpu_buffer_rsrc_t rsrc =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), 0, bytes, kBufferFlags);
#pragma unroll
        for (int j = 0; j < J; ++j)
            pre[d][i][j] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, 16 * lane + 1024 * j, 0, kNonTemporal);
    };
    int qb = 0, qp = 0;  // batch and pass of the next step to request
    find_rows(0);
#pragma unroll
    for (int d = 0; d < D; ++d) {
#pragma unroll
        for (int i = 0; i < RS; ++i) issue_row(d, qp, i);
        if (++qp == npass) { qp = 0; find_rows(++qb); }
    }

    // x into LDS once per workgroup (overlaps the first weight loads).
    in.stage(rows.input(0), xl, bpr, reinterpret_cast<float*>(lds_dyn + pipe_x_bytes(bpr)));

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    int cb = 0, cp = 0;  // current batch and pass
    for (int s0 = 0; s0 < steps; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int s = s0 + d;
            if (s >= steps) break;
            const int b0 = cp * LPR;
            const int nblk = min(LPR, bpr - b0);
            const int col = li < nblk ? b0 + li : 0;
            float xv[32];
            {
                const uint8_t* xs = xl + x_block_offset(col);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const f32x4 t = *reinterpret_cast<const f32x4*>(xs + 16 * i);
                    xv[4 * i + 0] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w;
                }
            }
#pragma unroll
            for (int it = 0; it < R; ++it) {
#pragma unroll
                for (int gg = 0; gg < G; ++gg) {
#pragma unroll
                    for (int j = 0; j < J; ++j)
                        *reinterpret_cast<u32x4*>(wl + gg * S::SEGP + 1024 * j + 16 * lane) = pre[d][it * G + gg][j];
                    issue_row(d, qp, it * G + gg);  // step s + D into the slot just emptied
                }
                wave_lds_sync();
                if (li < nblk) {
                    const uint32_t p = g * S::SEGP + li * BB;
                    acc[it] += Q4 ? block_dot_q4_exact(wl, p, xv) : block_dot_q8(wl, p, xv);
                }
                wave_lds_sync();
            }
            if (++qp == npass) { qp = 0; find_rows(++qb); }
            if (cp == npass - 1) {
                if constexpr (decltype(rows)::kSwiGLUPairs) {
                    // Iteration 0 is a gate row, iteration 1 its up row.
                    static_assert(R == 2 && G == 1, "SwiGLU pairs need two row iterations of one row group");
                    const float gate = group_sum<LPR>(acc[0]);
                    const float up = group_sum<LPR>(acc[1]);
                    const int row = gw + cb * RS * GW;
                    if (li == 0 && row < nrows) rows.store_pair(row, gate, up);
                    acc[0] = acc[1] = 0.0f;
                } else {
#pragma unroll
                    for (int it = 0; it < R; ++it) {
                        const float total = group_sum<LPR>(acc[it]);
                        const int row = gw + (cb * RS + it * G + g) * GW;
                        if (li == 0 && row < nrows) rows.store(row, rows.previous(row) + total);
                        acc[it] = 0.0f;
                    }
                }
            }
            if (++cp == npass) { cp = 0; ++cb; }
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

constexpr size_t kLdsPerCU = 160 * 1024;

// Streaming launch: persistent grid sized to what is resident at once on 256
// CUs -- workgroups of 4 (or 8) wavefronts, as many per CU as LDS allows (at
// most 2 of 4 or 1 of 8 = 8 wavefronts per CU, the occupancy that streams
// best) -- never more workgroups than row tiles need.
template <uint32_t QT, int LPR, int R, class Rows>
inline int launch_stream(const Rows& rows, int nrows, int bpr, int wpb, size_t lds, int wgs_per_cu,
                         hipStream_t stream) {
    using S = StagedShape<QT, LPR, R>;
    auto kernel = mv_stream_kernel<QT, LPR, R, Rows>;
    // Allow the largest dynamic LDS this instantiation can use (once per
    // process: the first call of each instantiation, typically eager).
    static const bool lds_ready =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(kLdsPerCU)) == hipSuccess;
    if (lds > 64 * 1024 && !lds_ready) return Q3X_HIP_ERUNTIME;
    const long long units = (nrows + S::RW - 1) / S::RW;
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

inline StreamPlan plan_stream(int wave_lds) {
    StreamPlan p;
    // 8 resident wavefronts per CU: one workgroup of 8 (measured slightly
    // ahead), else two of 4.
    if (8u * wave_lds <= kLdsPerCU) { p.wpb = 8; p.per_cu = 1; p.lds = 8u * wave_lds; p.ok = true; }
    else if (4u * wave_lds * 2 <= kLdsPerCU) { p.wpb = 4; p.per_cu = 2; p.lds = 4u * wave_lds; p.ok = true; }
    return p;
}

// Chooses R for LPR lanes per row: the cost of a candidate is the rows one
// wavefront streams -- ceil(tiles / waves) * rows per tile, so uneven tile
// counts are charged -- times the extra x traffic of small tiles.
template <uint32_t QT, int LPR, class Rows>
inline int launch_staged(const Rows& rows, int nrows, int bpr, hipStream_t stream) {
    const StreamPlan p4 = plan_stream(StagedShape<QT, LPR, 4>::WAVE_LDS);
    const StreamPlan p2 = plan_stream(StagedShape<QT, LPR, 2>::WAVE_LDS);
    const StreamPlan p1 = plan_stream(StagedShape<QT, LPR, 1>::WAVE_LDS);
    const bool q8 = QT == Q3X_HIP_MATRIX_Q8_0;
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
        return launch_stream<QT, LPR, 4>(rows, nrows, bpr, p4.wpb, p4.lds, p4.per_cu, stream);
    if (c2 <= c1 && p2.ok)
        return launch_stream<QT, LPR, 2>(rows, nrows, bpr, p2.wpb, p2.lds, p2.per_cu, stream);
    return launch_stream<QT, LPR, 1>(rows, nrows, bpr, p1.wpb, p1.lds, p1.per_cu, stream);
}

// Pipe launch: rows per step RS = G * R; a wave takes B batches, B the
// fewest that the resident waves allow, and the grid then shrinks so that
// every wave gets B full batches (balanced), spreading the waves over all
// CUs (fewer per workgroup) when there are fewer than 256 workgroups' worth.
template <uint32_t QT, int LPR, int R, class Rows, int D = 1, int WPE = 4, class In = PlainInput>
inline int launch_pipe(const Rows& rows, int nrows, int bpr, int wpb, hipStream_t stream, int per_cu = 1,
                       const In& in = In{}) {
    using S = PipeShape<QT, LPR>;
    auto kernel = mv_pipe_kernel<QT, LPR, R, D, Rows, WPE, In>;
    static const bool lds_ready =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(kLdsPerCU)) == hipSuccess;
    constexpr size_t tail = rows_route<Rows>::lds;
    size_t lds = pipe_x_bytes(bpr) + static_cast<size_t>(wpb) * S::WAVE_LDS + tail;
    while (lds > kLdsPerCU && wpb > 4) {
        wpb -= 4;
        lds = pipe_x_bytes(bpr) + static_cast<size_t>(wpb) * S::WAVE_LDS + tail;
    }
    if (lds > kLdsPerCU) return Q3X_HIP_ENOTSUP;  // x too long for LDS
    if (lds > 64 * 1024 && !lds_ready) return Q3X_HIP_ERUNTIME;
    if (lds * per_cu > kLdsPerCU) per_cu = 1;
    const long long rs = static_cast<long long>(S::G) * R;
    const long long gw_max = static_cast<long long>(kCUs) * per_cu * wpb;
    const long long batches = (nrows + gw_max * rs - 1) / (gw_max * rs);
    const long long waves =
        std::max<long long>((nrows + batches * rs - 1) / (batches * rs), rows.matrices());
    const int wpb_used = static_cast<int>(std::min<long long>(wpb, (waves + kCUs * per_cu - 1) / (kCUs * per_cu)));
    const int grid = static_cast<int>((waves + wpb_used - 1) / wpb_used);
    lds = pipe_x_bytes(bpr) + static_cast<size_t>(wpb_used) * S::WAVE_LDS + tail;
    Rows planned = rows;
    planned.plan_waves(grid * wpb_used);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kWave * wpb_used), lds, stream, planned, nrows, bpr, in);
    return launch_status();
}

// Shapes measured on MI355X (rows per step x waves per workgroup x
// workgroups per CU x prefetch depth): Q8_0 streams best with one row per
// step; Q4_0, whose rows are half as long, with two; large matrices gain from
// a grid of two 16-wave workgroups per CU (more, shorter waves: the grid
// drains evenly).  Prefetching two or three steps ahead measured slower at
// every size (the registers cost more occupancy than the extra bytes in
// flight gain), so the launches use one.
template <uint32_t QT, class Rows, class In = PlainInput>
inline int launch_pipe_for(const Rows& rows, int nrows, int bpr, hipStream_t stream, const In& in = In{}) {
    if (bpr <= 16) return launch_pipe<QT, 16, 1, Rows, 1, 4, In>(rows, nrows, bpr, 16, stream, 1, in);
    if (bpr <= 32) return launch_pipe<QT, 32, 1, Rows, 1, 4, In>(rows, nrows, bpr, 16, stream, 1, in);
    if (QT == Q3X_HIP_MATRIX_Q8_0) {
        // 8K-64K rows (a fused q|k|v or qkv|z|a|b projection, a gate|up
        // pair): a 64-VGPR build, so that two 16-wave workgroups are resident
        // per CU (the default build needs 68 VGPRs, 7 waves per SIMD, which
        // leaves room for one); 12% faster than the default build at 14K
        // rows.  Taller matrices stream as well without it.
        if (nrows >= 8192 && nrows <= 65536)
            return launch_pipe<QT, 64, 1, Rows, 1, 8, In>(rows, nrows, bpr, 16, stream, 2, in);
        return launch_pipe<QT, 64, 1, Rows, 1, 4, In>(rows, nrows, bpr, 16, stream, nrows >= 8192 ? 2 : 1, in);
    }
    // Short Q4_0 rows that 64-block passes would leave partly idle (e.g. 160
    // blocks = 2.5 passes) take 32 lanes per row (two rows per pass).  The
    // lanes per row depend on the row length only, so the per-row reduction
    // order (and the result) is the same whatever the launch's row count.
    // The two-row build needs 70 VGPRs (7 waves per SIMD), so one 16-wave
    // workgroup per CU is resident: a grid of one per CU (each wave twice the
    // rows) avoids a second round of workgroups.  At 34816 x 160 blocks it
    // takes 23.0 us against 24.3 us for one row per step on two workgroups
    // per CU (60 VGPRs; interleaved A/B, medians of 9 rounds).
    if (bpr <= 256 && bpr % 64 != 0 && bpr % 32 == 0) {
        if (nrows <= 4096) return launch_pipe<QT, 32, 1, Rows, 1, 4, In>(rows, nrows, bpr, 16, stream, 1, in);
        return launch_pipe<QT, 32, 2, Rows, 1, 4, In>(rows, nrows, bpr, 16, stream, 1, in);
    }
    if (nrows <= 4096) return launch_pipe<QT, 64, 1, Rows, 1, 4, In>(rows, nrows, bpr, 16, stream, 1, in);
    return launch_pipe<QT, 64, 2, Rows, 1, 4, In>(rows, nrows, bpr, 16, stream, 2, in);
}

template <uint32_t QT, class Rows>
int launch_mv(const Rows& rows, int nrows, int bpr, bool staged, hipStream_t stream) {
    if (!staged) {
        const int grid = (nrows + kMvWaves - 1) / kMvWaves;
        hipLaunchKernelGGL((mv_generic_kernel<QT, Rows>), dim3(grid), dim3(kMvWaves * kWave), 0,
                           stream, rows, nrows, bpr);
        return launch_status();
    }
    // x shared by all rows and short enough for LDS: the pipelined kernel;
    // otherwise the streaming kernel reading x per unit from global memory.
    int status = Q3X_HIP_ENOTSUP;
    if constexpr (Rows::kSharedInput) status = launch_pipe_for<QT>(rows, nrows, bpr, stream);
    if (status != Q3X_HIP_ENOTSUP) return status;
    if (bpr <= 16) return launch_staged<QT, 16>(rows, nrows, bpr, stream);
    if (bpr <= 32) return launch_staged<QT, 32>(rows, nrows, bpr, stream);
    return launch_staged<QT, 64>(rows, nrows, bpr, stream);
}

constexpr float kEps = 1e-6f;  // RMSNorm epsilon, engine.cpp:26 EPS

__device__ __forceinline__ float bf16_value(uint16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }

// Input staging for a decode step's projections (mv_pipe_kernel's `In`):
// x = RMSNorm(h) * (1 + w) of the raw residual h (engine.cpp:228-233),
// formed by every workgroup of the matvec launch on its way into LDS.  Each
// thread loads its 16-byte chunks of h together with their four norm
// weights (one round trip; the first kHeld chunks stay in registers) and
// copies h to LDS; after one barrier wave 0 sums the squares of all of h
// from LDS in one fixed order (lane l takes chunks l, l + 64, ... with FMAs,
// then the wave's DPP tree), so every workgroup -- whatever the launch shape
// -- forms the same scale, and hands it to the other waves through LDS; then
// each thread scales its own chunks.  Requires w 8-byte aligned.
struct NormInput {
    static constexpr int kHeld = 4;
    const uint16_t* w;
    __device__ void stage(const float* x, uint8_t* xl, int bpr, float* work) const {
        const int chunks = bpr * 8;
        const int B = blockDim.x;
        const f32x4* xs = reinterpret_cast<const f32x4*>(x);
        const uint2* ws = reinterpret_cast<const uint2*>(w);
        auto at = [&](int c) { return reinterpret_cast<f32x4*>(xl + x_block_offset(c >> 3) + 16 * (c & 7)); };
        f32x4 xr[kHeld];
        uint2 wr[kHeld];
#pragma unroll
        for (int k = 0; k < kHeld; ++k) {
            const int c = threadIdx.x + k * B;
            if (c < chunks) {
                xr[k] = xs[c];
                wr[k] = ws[c];
            }
        }
#pragma unroll
        for (int k = 0; k < kHeld; ++k) {
            const int c = threadIdx.x + k * B;
            if (c < chunks) *at(c) = xr[k];
        }
        for (int c = threadIdx.x + kHeld * B; c < chunks; c += B) *at(c) = xs[c];
        __syncthreads();
        // Wave 0 alone sums the squares and hands the scale to the other
        // waves through LDS (a sum in every wave would read all of h from
        // LDS 16 times over).
        if (threadIdx.x < kWave) {
            float square = 0.0f;
            for (int c = threadIdx.x; c < chunks; c += kWave) {
                const f32x4 v = *at(c);
                square = fmaf(v.x, v.x, square);
                square = fmaf(v.y, v.y, square);
                square = fmaf(v.z, v.z, square);
                square = fmaf(v.w, v.w, square);
            }
            const float total = wave_sum_f32(square);
            if (threadIdx.x == 0) work[0] = 1.0f / sqrtf(total / static_cast<float>(bpr * kBlock) + kEps);
        }
        __syncthreads();  // the scale is in LDS; every read of h for it precedes the scaled writes
        const float scale = work[0];
        auto put = [&](int c, f32x4 v, uint2 q) {
            v.x = v.x * scale * (1.0f + bf16_value(static_cast<uint16_t>(q.x)));
            v.y = v.y * scale * (1.0f + bf16_value(static_cast<uint16_t>(q.x >> 16)));
            v.z = v.z * scale * (1.0f + bf16_value(static_cast<uint16_t>(q.y)));
            v.w = v.w * scale * (1.0f + bf16_value(static_cast<uint16_t>(q.y >> 16)));
            *at(c) = v;
        };
#pragma unroll
        for (int k = 0; k < kHeld; ++k) {
            const int c = threadIdx.x + k * B;
            if (c < chunks) put(c, xr[k], wr[k]);
        }
        for (int c = threadIdx.x + kHeld * B; c < chunks; c += B) put(c, *at(c), ws[c]);
        __syncthreads();
    }
};

}  // namespace q3x

