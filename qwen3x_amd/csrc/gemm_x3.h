// gemm_x3.h -- FP32 GEMM with exact products on the bf16 matrix cores.
//
// Y[m, n] = sum over blocks b of d[n, b] * (sum over the block's 32 k of
// A[m, k] q[n, k]): the reference's per-block factorisation of a quantized
// dot (arch/cpu.cpp:64-73, 91-106), for A in FP32 and q the block's integers
// (Q8_0: int8, Q4_0: nibble - 8), or for BF16 weights a plain sum over K
// (engine.cpp:181-185).
//
// Every weight value q is exact in bf16 (at most 8 significant bits), and an
// FP32 activation splits exactly into three bf16 values, a = a1 + a2 + a3:
// a1 is a truncated to its upper 16 bits, a2 the remainder truncated the
// same way, a3 what is left (at most 8 significant bits; both subtractions
// are exact by Sterbenz's lemma).  So
//   sum_k a q = sum_k a3 q + sum_k a2 q + sum_k a1 q,
// three v_mfma_f32_16x16x32_bf16 per 16x16 output block and weight block,
// each product exact and every sum in FP32 -- where the FP32 matrix
// instruction (v_mfma_f32_16x16x4_f32) needs eight instructions of twice the
// cycles for the same block.  The split is exact for |a| >= 2^-110; below,
// the lowest part loses bits under 2^-133 (bf16 has 8 significant bits in
// FP32's subnormal range), an absolute error far below the FP32 rounding of
// any sum it enters.
//
// KS = 2 runs the tile on two groups of WM x WN waves, each over half of the
// K blocks (the first half the first ceil(blocks / 2)) with its own LDS
// buffers; the second group's sums then pass through LDS and the first adds
// them, acc = first + second, a fixed order.
//
// Tile: WM x WN waves, each SM x SN output blocks of 16x16 (wave tile
// 16 SM x 16 SN); BM = 16 SM WM A rows, BN = 16 SN WN weight rows.  A K
// stage is one weight block (32 columns).  Per stage the workgroup stages,
// in LDS, the three bf16 planes of its A rows (split once per tile) and its
// weight rows as bf16, 64 bytes a row, the 16-byte chunks of row r at
// position chunk ^ ((r >> 1) & 3), so the operand reads (lane l: row l % 16,
// chunk l / 16) of each eight consecutive rows fall on distinct banks.  Per
// stage kb: stage kb + 1 goes from registers to the other LDS buffer (the
// previous barrier freed it), the loads of stage kb + 1 + PF are issued
// into the registers just emptied, the matrix instructions of stage kb run,
// then one barrier; at the LDS write the only loads in flight are the ones
// it consumes, so the wait is exact.  Past the last block the store and the
// loads repeat the last block (into a buffer no stage reads), so a step has
// no branch.  CF ("compute first") issues stage kb's matrix instructions
// before stage kb + 1's conversion instead, so the scheduler places the
// split and the weight conversion in the matrix instructions' shadow; with
// two stages of loads ahead it measures 1-4% slower on 64x64 wave tiles and
// on 32x32 ones it costs a wave of occupancy; the grouped MoE GEMMs' 80x32
// wave tiles keep their occupancy with it and use it.
//
// A policy supplies the tiles and the operand rows: tile(ty, BM, tile)
// (false: no such tile), a_row(tile, m) (an FP32 A row), b_row(tile, n) (a
// weight row), store(tile, m, n, v) or, with kPairedColumns,
// store_pair(tile, m, n, v, v16) for columns n and n + 16; kLinearGrid (a
// 1-D grid of tiles_x weight-row tiles per A tile, remapped so that each
// XCD takes a contiguous run: workgroups that share an A tile share an L2;
// optionally linear_total()); kPartialTiles (A tiles often short).  With
// kPartialTiles the wave's subtile rows are the tile's rows 16 (i WM + wm)
// + [0, 16), so the valid rows of a short tile spread over the wave rows,
// and a wave skips the subtile rows past the valid ones.
#pragma once

#include "gemm.h"

namespace q3x {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// LDS byte offset of 16-byte chunk c (0..3) of row r in a 64-byte-row tile.
__device__ __forceinline__ int x3_offset(int r, int c) { return r * 64 + 16 * (c ^ ((r >> 1) & 3)); }

// The upper halves of two words as one word of two bf16: lo from x, hi from y.
__device__ __forceinline__ uint32_t bf16_pair(uint32_t x, uint32_t y) {
    return __builtin_amdgcn_perm(y, x, 0x07060302u);
}

// a = a1 + a2 + a3 exactly (|a| >= 2^-110): each part's word has its low
// half zero, i.e. is a bf16 value in the upper half.
__device__ __forceinline__ void split3(float a, uint32_t& h1, uint32_t& h2, uint32_t& h3) {
    h1 = __float_as_uint(a) & 0xffff0000u;
    const float r = a - __uint_as_float(h1);
    h2 = __float_as_uint(r) & 0xffff0000u;
    h3 = __float_as_uint(r - __uint_as_float(h2));
}

// K split over workgroups (policies with ksplit and part members, e.g. a
// GEMM given a workspace): the launch has ksplit units per tile, unit s
// taking the tile's K blocks [s * per, (s + 1) * per), per = ceil(blocks /
// ksplit); each unit writes its sums, as its threads hold them, to its slot
// of `part`, and gemm_x3_fixup_kernel adds a tile's units in K order and
// stores.  So a launch of few tiles over long K (512 tokens x 5120 rows x
// 17408 columns is 80 tiles of 128 x 256 for 256 CUs) fills the chip;
// results are deterministic, their sums in another order than unsplit.
template <class P, class = void>
struct KSplit {
    __device__ static int count(const P&) { return 1; }
    __device__ static float* part(const P&) { return nullptr; }
};
template <class P>
struct KSplit<P, decltype(void(std::declval<const P&>().ksplit))> {
    __device__ static int count(const P& p) { return p.ksplit; }
    __device__ static float* part(const P& p) { return p.part; }
};

// Floats of one unit's partial sums: every thread's SM x SN x 4 values.
template <int WM, int WN, int SM, int SN>
constexpr size_t x3_unit_floats() { return static_cast<size_t>(SM) * SN * 4 * WM * WN * kWave; }

// The tile's stores: output block (i, j) of wave (wm, wn), lane rows
// 4 g16 + e, column l16.
template <int WM, int WN, int SM, int SN, class Policy>
__device__ __forceinline__ void x3_store(const Policy& pol, const GemmTile& tile, int n0, int rows, int wm,
                                         int wn, int l16, int g16, int nsub, const f32x4 (&acc)[SM][SN]) {
#pragma unroll
    for (int i = 0; i < SM; ++i) {
        if (i >= nsub) break;
        const int row0 = 16 * (i * WM + wm);
#pragma unroll
        for (int j = 0; j < SN; ++j) {
            const int n = n0 + (wn * SN + j) * 16 + l16;
            if constexpr (Policy::kPairedColumns) {
                // Column blocks 2s and 2s + 1 hold columns q and q + 16 of a
                // 32-column group (e.g. gate and up of one output feature).
                if (j % 2 == 1) continue;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = row0 + 4 * g16 + e;
                    if (m < tile.mcount && n < rows) pol.store_pair(tile, m, n, acc[i][j][e], acc[i][j + 1][e]);
                }
            } else {
                if (n >= rows) continue;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = row0 + 4 * g16 + e;
                    if (m < tile.mcount) pol.store(tile, m, n, acc[i][j][e]);
                }
            }
        }
    }
}

template <uint32_t QT, int WM, int WN, int SM, int SN, class Policy, int PF = 1, bool CF = false, int KS = 1>
__global__ __launch_bounds__(KS * WM * WN * kWave) void gemm_x3_kernel(Policy pol, int rows, int cols) {
    static_assert(PF == 1 || PF == 2, "one or two stages in flight");
    static_assert(KS == 1 || KS == 2, "the K blocks in one or two halves");
    static_assert(!Policy::kPairedColumns || SN % 2 == 0, "paired columns need column blocks in pairs");
    constexpr int NT = WM * WN * kWave;  // threads of one K half
    constexpr int BM = WM * SM * 16;
    constexpr int BN = WN * SN * 16;
    constexpr int BB = QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : QT == Q3X_HIP_MATRIX_Q4_0 ? kQ4Bytes : kBF16Bytes;
    constexpr bool kScaled = QT != Q3X_HIP_MATRIX_BF16;
    // A: BM rows x 8 float4 per stage.
    constexpr int A_VEC = BM * 8;
    constexpr int A_PER_T = (A_VEC + NT - 1) / NT;
    // Weights: BN rows, PARTS threads per row.
    constexpr int PARTS = NT / BN >= 2 ? 2 : 1;
    constexpr int B_ROWS_PER_PASS = NT / PARTS;
    constexpr int B_PASSES = (BN + B_ROWS_PER_PASS - 1) / B_ROWS_PER_PASS;
    constexpr int PER_PART = 32 / PARTS;
    static_assert(PARTS * B_ROWS_PER_PASS == NT, "thread split");
    using Part = BlockPart<QT, PARTS>;

    // One LDS buffer: the A planes (a1, a2, a3), the weight rows, the scales.
    constexpr int A_BYTES = BM * 64, B_BYTES = BN * 64, D_BYTES = kScaled ? BN * 4 : 0;
    constexpr int BUF = 3 * A_BYTES + B_BYTES + D_BYTES;
    __shared__ __attribute__((aligned(16))) uint8_t lds_all[KS * 2 * BUF];
    // With KS = 2 the second half's partial sums come back through LDS.
    static_assert(KS == 1 || SM * SN * 4 * 4 * NT <= 2 * BUF, "partials fit a half's buffers");
    const int half = KS == 1 ? 0 : __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / NT);
    uint8_t* const lds = lds_all + half * 2 * BUF;
    auto plane = [&](int buf, int p) { return lds + buf * BUF + p * A_BYTES; };
    auto wtile = [&](int buf) { return lds + buf * BUF + 3 * A_BYTES; };
    auto scales = [&](int buf) { return reinterpret_cast<float*>(lds + buf * BUF + 3 * A_BYTES + B_BYTES); };
    // The weight values' chunk order (BlockPart's columns: for Q4_0 with two
    // parts, elements 0-7 | 16-23 | 8-15 | 24-31); A's elements take the
    // same chunks, so the products pair up unchanged.
    auto a_chunk = [](int c) {
        if constexpr (QT == Q3X_HIP_MATRIX_Q4_0 && PARTS == 2) return c == 1 ? 2 : c == 2 ? 1 : c;
        else return c;
    };

    // Units of a split launch are numbered split-major (unit = split *
    // tiles + tile), so an XCD's contiguous run shares its A tile's K range.
    const int S = KSplit<Policy>::count(pol);
    int bx = blockIdx.x, by = blockIdx.y, split = 0, tile_id = 0;
    if constexpr (Policy::kLinearGrid) {
        const int total = LinearTotal<Policy>::get(pol, gridDim.x), L = blockIdx.x;
        if (L >= total) return;
        const int q = total / kXcds, r = total % kXcds, xcd = L % kXcds, k = L / kXcds;
        int t = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + k;
        if (S > 1) {
            const int tiles = total / S;
            split = t / tiles;
            t %= tiles;
        }
        tile_id = t;
        bx = t % pol.tiles_x;
        by = t / pol.tiles_x;
    }
    GemmTile tile;
    if (!pol.tile(by, BM, tile)) return;
    const int n0 = bx * BN;
    const int tid = static_cast<int>(threadIdx.x) % NT;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int wm = wave / WN, wn = wave % WN;
    const int l16 = lane & 15, g16 = lane >> 4;

    // Source pointers, fixed over K.  Every thread loads every stage with no
    // branch (rows past the valid A rows or past the matrix read a valid row
    // instead; their outputs are never stored).
    const float* a_src[A_PER_T];
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
        const int idx = min(tid + i * NT, A_VEC - 1);
        a_src[i] = pol.a_row(tile, min(idx >> 3, tile.mcount - 1)) + 4 * (idx & 7);
    }
    const uint8_t* b_src[B_PASSES];
    const int b_part = tid % PARTS;
#pragma unroll
    for (int p = 0; p < B_PASSES; ++p) {
        const int n = min(tid / PARTS + p * B_ROWS_PER_PASS, BN - 1);
        b_src[p] = pol.b_row(tile, min(n0 + n, rows - 1));
    }

    // The K blocks of this half: [kbeg, kbeg + kcnt); both halves run
    // kmax stages (the same barriers), a half past its own count computes
    // nothing.
    const int nblk_all = cols / kBlock;
    const int per = (nblk_all + S - 1) / S;                 // the unit's K blocks
    const int ubeg = split * per, ucnt = min(per, nblk_all - ubeg);
    const int kmax = (ucnt + KS - 1) / KS;
    const int kbeg = ubeg + half * kmax;
    const int kcnt = KS == 1 ? ucnt : min(kmax, ubeg + ucnt - kbeg);
    f32x4 a_reg[PF][A_PER_T];
    uint32_t b_raw[PF][B_PASSES][1 + Part::WORDS];
    auto load_stage = [&](int kb, int r) {
        const int k = min(kbeg + max(kb, 0), nblk_all - 1);
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) a_reg[r][i] = *reinterpret_cast<const f32x4*>(a_src[i] + 32 * k);
#pragma unroll
        for (int p = 0; p < B_PASSES; ++p) Part::load(b_src[p] + static_cast<size_t>(k) * BB, b_part, b_raw[r][p]);
    };
    auto store_stage = [&](int buf, int r) {
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            const int idx = tid + i * NT;
            if (A_VEC % NT == 0 || idx < A_VEC) {
                const int row = idx >> 3, q4 = idx & 7;
                const int off = x3_offset(row, a_chunk(q4 >> 1)) + 8 * (q4 & 1);
                uint32_t h[3][4];
#pragma unroll
                for (int e = 0; e < 4; ++e) split3(a_reg[r][i][e], h[0][e], h[1][e], h[2][e]);
#pragma unroll
                for (int p = 0; p < 3; ++p)
                    *reinterpret_cast<uint2*>(plane(buf, p) + off) =
                        uint2{bf16_pair(h[p][0], h[p][1]), bf16_pair(h[p][2], h[p][3])};
            }
        }
#pragma unroll
        for (int p = 0; p < B_PASSES; ++p) {
            const int n = tid / PARTS + p * B_ROWS_PER_PASS;
            if (BN % B_ROWS_PER_PASS == 0 || n < BN) {
                uint32_t w[PER_PART / 2];
                if constexpr (kScaled) {
                    uint32_t raw[1 + Part::WORDS];
#pragma unroll
                    for (int i = 0; i <= Part::WORDS; ++i) raw[i] = b_raw[r][p][i];
                    Part::finish(raw, b_part);
                    float vals[PER_PART];
                    Part::values(raw, vals);
#pragma unroll
                    for (int e = 0; e < PER_PART / 2; ++e)
                        w[e] = bf16_pair(__float_as_uint(vals[2 * e]), __float_as_uint(vals[2 * e + 1]));
                    scales(buf)[n] = Part::scale(raw);  // the row's parts write the same value
                } else {
#pragma unroll
                    for (int e = 0; e < PER_PART / 2; ++e) w[e] = b_raw[r][p][1 + e];  // two bf16 a word already
                }
#pragma unroll
                for (int c = 0; c < PER_PART / 8; ++c)
                    *reinterpret_cast<u32x4*>(wtile(buf) + x3_offset(n, (b_part * PER_PART) / 8 + c)) =
                        u32x4{w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]};
            }
        }
    };

    // acc[i][j]: output block (subtile row i, column block j); lane l holds
    // rows 4 (l / 16) + r, column l % 16.
    f32x4 acc[SM][SN];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto sub_row = [&](int i) { return 16 * (i * WM + wm); };
    const int s16 = (tile.mcount + 15) / 16;
    const int nsub = Policy::kPartialTiles ? max(0, min(SM, (s16 - wm + WM - 1) / WM)) : SM;
    const bool active = nsub > 0;
    const int nblk = kcnt;

    auto step = [&](int kb, int r) {
        const int buf = kb & 1;
        if constexpr (!CF) {
            store_stage(buf ^ 1, r);
            load_stage(min(kb + 1 + PF, nblk - 1), r);
        }
        if (active && (KS == 1 || kb < nblk)) {
            bf16x8 bf[SN];
            float d[SN];
#pragma unroll
            for (int j = 0; j < SN; ++j) {
                const int n = (wn * SN + j) * 16 + l16;
                bf[j] = *reinterpret_cast<const bf16x8*>(wtile(buf) + x3_offset(n, g16));
                if constexpr (kScaled) d[j] = scales(buf)[n];
            }
#pragma unroll
            for (int i = 0; i < SM; ++i) {
                if (i >= nsub) break;
                const int m = sub_row(i) + l16;
                const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(plane(buf, 0) + x3_offset(m, g16));
                const bf16x8 a2 = *reinterpret_cast<const bf16x8*>(plane(buf, 1) + x3_offset(m, g16));
                const bf16x8 a3 = *reinterpret_cast<const bf16x8*>(plane(buf, 2) + x3_offset(m, g16));
#pragma unroll
                for (int j = 0; j < SN; ++j) {
                    if constexpr (kScaled) {
                        // The block's sum from zero, smallest parts first,
                        // then acc = fma(d, sum, acc).
                        f32x4 s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, bf[j], f32x4{0.0f, 0.0f, 0.0f, 0.0f},
                                                                          0, 0, 0);
                        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bf[j], s, 0, 0, 0);
                        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bf[j], s, 0, 0, 0);
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf(d[j], s[e], acc[i][j][e]);
                    } else {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, bf[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bf[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bf[j], acc[i][j], 0, 0, 0);
                    }
                }
            }
        }
        if constexpr (CF) {
            store_stage(buf ^ 1, r);
            load_stage(min(kb + 1 + PF, nblk - 1), r);
        }
        __syncthreads();
    };
    // Prologue: stage 0 into LDS buffer 0, stages 1..PF into registers.
    load_stage(0, 0);
    store_stage(0, 0);
#pragma unroll
    for (int q = 1; q <= PF; ++q) load_stage(min(q, nblk - 1), q % PF);
    __syncthreads();
    // Stage s + 1 is in register set (s + 1) % PF when stage s runs.
    const int nsteps = KS == 1 ? nblk : kmax;
    for (int kb = 0; kb < nsteps; kb += 2) {
        step(kb, PF == 1 ? 0 : 1);
        if (kb + 1 < nsteps) step(kb + 1, 0);
    }
    if constexpr (KS == 2) {
        // The second half's sums to LDS (its own buffers, free after the
        // last barrier), then the first half adds them: acc = first + second.
        float* part = reinterpret_cast<float*>(lds_all + 2 * BUF);
        if (half == 1) {
#pragma unroll
            for (int i = 0; i < SM; ++i)
#pragma unroll
                for (int j = 0; j < SN; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) part[((i * SN + j) * 4 + e) * NT + tid] = acc[i][j][e];
        }
        __syncthreads();
        if (half == 1) return;
#pragma unroll
        for (int i = 0; i < SM; ++i)
#pragma unroll
            for (int j = 0; j < SN; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[i][j][e] += part[((i * SN + j) * 4 + e) * NT + tid];
    }

    if (S > 1) {
        // This unit's sums to its slot (coalesced: value v of thread t at
        // v * NT + t); the fixup adds the tile's units and stores.
        float* slot = KSplit<Policy>::part(pol) +
                      (static_cast<size_t>(tile_id) * S + split) * x3_unit_floats<WM, WN, SM, SN>();
#pragma unroll
        for (int i = 0; i < SM; ++i)
#pragma unroll
            for (int j = 0; j < SN; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) slot[((i * SN + j) * 4 + e) * NT + tid] = acc[i][j][e];
        return;
    }
    x3_store<WM, WN, SM, SN>(pol, tile, n0, rows, wm, wn, l16, g16, nsub, acc);
}

// The stores of a split launch, one output value per thread: value f (in
// the units' layout, f = v * NT + t for value v of thread t) of tile
// blockIdx.x / (BM * BN / 256), its units added in K order (unit 0 first),
// stored where gemm_x3_kernel's thread t would store its value v.  With
// kPairedColumns the thread of an even column block stores the pair, its
// partner's value (column block j + 1, the same lane, row and e) summed the
// same way, and the thread of the odd block stores nothing.
template <int WM, int WN, int SM, int SN, class Policy>
__global__ __launch_bounds__(256) void gemm_x3_fixup_kernel(Policy pol, int rows) {
    constexpr int NT = WM * WN * kWave;
    constexpr int BM = WM * SM * 16, BN = WN * SN * 16;
    constexpr int U = static_cast<int>(x3_unit_floats<WM, WN, SM, SN>());  // BM * BN
    static_assert(U % 256 == 0, "whole workgroups per tile");
    constexpr int kPerTile = U / 256;
    const int t = blockIdx.x / kPerTile;
    const int f = (blockIdx.x % kPerTile) * 256 + threadIdx.x;
    GemmTile tile;
    if (!pol.tile(t / pol.tiles_x, BM, tile)) return;
    const int S = pol.ksplit;
    const float* units = pol.part + static_cast<size_t>(t) * S * U;
    auto unit_sum = [&](int g) {
        float sum = units[g];
        for (int u = 1; u < S; ++u) sum += units[static_cast<size_t>(u) * U + g];
        return sum;
    };
    const int v = f / NT, tid = f % NT;
    const int i = v / (SN * 4), j = (v / 4) % SN, e = v % 4;
    const int lane = tid & (kWave - 1), wave = tid / kWave;
    const int wm = wave / WN, wn = wave % WN, l16 = lane & 15, g16 = lane >> 4;
    const int m = 16 * (i * WM + wm) + 4 * g16 + e;
    const int n = (t % pol.tiles_x) * BN + (wn * SN + j) * 16 + l16;
    if (m >= tile.mcount || n >= rows) return;
    if constexpr (Policy::kPairedColumns) {
        static_assert(SN % 2 == 0, "paired columns need column blocks in pairs");
        if (j % 2 == 0) pol.store_pair(tile, m, n, unit_sum(f), unit_sum(f + 4 * NT));
    } else {
        pol.store(tile, m, n, unit_sum(f));
    }
}

// Tile shapes of the launches: 128 A rows x 256 weight rows on 8 waves of
// 64x64 (one workgroup per CU: 209 registers), 128 x 192 on 8 waves of
// 64x48 (one per CU; paired-column policies excluded: SN is odd), 64 x 128
// on 8 waves of 32x32 (three), 64 x 64 on 4 waves of 32x32 (four).  128 x 192
// exists for row counts that 256 leaves uneven over the CUs: 512 tokens x
// 12288 rows x 4096 columns is 256 tiles of it, one per CU, at 306 TFLOP/s
// (Q8_0; 260 on 128 x 256, whose 192 tiles leave 64 CUs idle), and 512 x
// 17408 x 5120 runs at 257 (238 on 64 x 128); with many tiles per CU it
// runs at ~340, below 128 x 256's ~383.  Over long K (>= kX3LongK) a
// 64 x 128 tile can also run on two halves of 8 waves, each over half the
// K blocks with its own LDS buffers, the second half's sums added to the
// first's at the end (KS = 2; one 1024-thread workgroup per CU): 512 x 4096
// x 12288 is 256 such tiles, one per CU, at 233 (Q8_0) / 260 (Q4_0) TFLOP/s
// against 178 / 212 with 8 waves over the whole K; with more tiles than CUs
// it loses to the 8-wave tile (three resident).  (128 x 128 on 8 waves of
// 64x32, two per CU, measured 200 / 330 TFLOP/s at one / two resident and
// never beat these three on the config and engine shapes.)  A launch takes the shape of least estimated time: the
// busiest CU takes ceil(tiles / CUs) tiles, resident up to the occupancy at
// a time, and a CU holding k of them runs at the shape's measured rate for
// k (TFLOP/s over the chip, MI355X, dense Q8_0/Q4_0).  Measured, e.g.: 4096
// tokens x 12288 rows x 4096 columns 370 TFLOP/s on 128 x 256; 512 x 4096
// x 12288 (64 tiles of 128 x 256) 208 on 64 x 128; 512 x 17408 x 5120 253
// on 64 x 128 (272 tiles of 128 x 256 would leave 16 CUs a second one).
enum class X3Shape { k128x256, k64x128, k64x64, k128x192, k64x128_split };

// Per-CU time of `tiles` tiles (or units) of `area` outputs each (in units
// of area / (TFLOP/s): multiply by 2 K 256 / 1e12 for seconds).
inline double x3_estimate(long long tiles, double area, int occupancy, const double* rate) {
    long long left = (tiles + kCUs - 1) / kCUs;
    double t = 0.0;
    while (left > 0) {
        const int k = static_cast<int>(left < occupancy ? left : occupancy);
        t += k * area / rate[k - 1];
        left -= k;
    }
    return t;
}

// Two stages of loads ahead for the 64 x 128 tiles over long K (5-10% on
// 512 tokens x 12288- and 17408-column matrices, a few % slower on short K).
constexpr int kX3LongK = 8192;

// A launch: the tile shape and the units per tile of a K split (1: none).
struct X3Plan {
    X3Shape shape;
    int split;
    long long tiles;
    int bm, bn;
    size_t workspace_bytes() const { return split > 1 ? static_cast<size_t>(tiles) * split * bm * bn * 4 : 0; }
};

// The plan of least estimated time for rows weight rows, count A rows and
// K = cols; splits only where their partial sums fit `workspace` bytes.
// A split unit runs the tile shape over K / split blocks at the shape's
// rate, plus a per-round cost for its shorter pipeline (prologue, drain and
// the partial-sum stores), and the launch adds the fixup: the units' sums
// read back and the outputs written, and one more launch.
inline X3Plan x3_plan(int rows, int count, int cols, bool paired, size_t workspace) {
    auto tiles = [&](int bm, int bn) {
        return static_cast<long long>((rows + bn - 1) / bn) * ((count + bm - 1) / bm);
    };
    static constexpr double r256[] = {370.0};
    static constexpr double r64x128[] = {210.0, 240.0, 260.0};
    static constexpr double r64x128_long[] = {215.0, 290.0, 300.0};  // two stages ahead, K >= kX3LongK
    static constexpr double r64[] = {150.0, 190.0, 215.0, 230.0};
    static constexpr double r192[] = {300.0};
    static constexpr double r64x128_split[] = {240.0};  // K halves on 16 waves, one workgroup per CU
    struct Option {
        X3Shape shape;
        int bm, bn, occupancy;
        const double* rate;
        bool ok;
    };
    const bool long_k = cols >= kX3LongK;
    const Option options[5] = {
        {X3Shape::k128x256, 128, 256, 1, r256, true},
        {X3Shape::k64x128, 64, 128, 3, long_k ? r64x128_long : r64x128, true},
        {X3Shape::k64x64, 64, 64, 4, r64, true},
        {X3Shape::k128x192, 128, 192, 1, r192, !paired},
        {X3Shape::k64x128_split, 64, 128, 1, r64x128_split, long_k},
    };
    const int blocks = cols / kBlock;
    // Fitted to a sweep of every shape at splits 1, 2, 3, 4, 6 and 8 on six
    // prefill shapes (512 and 2048 tokens, 4096-17408 columns): the fit's
    // choice is within 2% of the fastest on each.  A unit's pipeline fill and
    // drain cost per round (less where other resident units hide them), and
    // the fixup's traffic moves at about a quarter of HBM's peak.
    constexpr double kRoundSeconds = 3e-6, kRoundSecondsShared = 2e-6;
    constexpr double kFixupBytesPerSecond = 2e12;
    constexpr double kLaunchSeconds = 5e-6;
    constexpr int kSplits[] = {1, 2, 3, 4, 6, 8};
    X3Plan best{X3Shape::k128x256, 1, 0, 128, 256};
    double best_t = 1e300;
    for (const Option& o : options) {
        if (!o.ok) continue;
        const long long t = tiles(o.bm, o.bn);
        const double area = static_cast<double>(o.bm) * o.bn;
        for (const int split : kSplits) {
            const int per = (blocks + split - 1) / split;
            if (split > 1 && (per < 8 || (split - 1) * per >= blocks)) continue;
            const X3Plan plan{o.shape, split, t, o.bm, o.bn};
            if (plan.workspace_bytes() > workspace) continue;
            double sec = x3_estimate(t * split, area / split, o.occupancy, o.rate) * 2.0 * cols * kCUs / 1e12;
            if (split > 1) {
                const long long rounds = (t * split + static_cast<long long>(kCUs) * o.occupancy - 1) /
                                         (static_cast<long long>(kCUs) * o.occupancy);
                sec += rounds * (o.occupancy == 1 ? kRoundSeconds : kRoundSecondsShared) + kLaunchSeconds +
                       static_cast<double>(t) * area * 4.0 * (split + 1) / kFixupBytesPerSecond;
            }
            if (sec < best_t) {
                best_t = sec;
                best = plan;
            }
        }
    }
    return best;
}

inline X3Shape x3_shape(int rows, int count, int cols, bool paired = false) {
    return x3_plan(rows, count, cols, paired, 0).shape;
}

template <class P, class = void>
struct HasKSplit : std::false_type {};
template <class P>
struct HasKSplit<P, decltype(void(std::declval<P&>().ksplit))> : std::true_type {};

// One launch of gemm_x3_kernel over count A rows (pol.count) and `rows`
// weight rows, on a 1-D grid (Policy::kLinearGrid) of all tiles (units);
// with split > 1 (policies with a workspace), the fixup launch follows.
template <uint32_t QT, int WM, int WN, int SM, int SN, int PF, bool CF, class P, int KS = 1>
int launch_x3_tiles(P pol, int rows, int count, int cols, hipStream_t stream, int split = 1) {
    constexpr int BM = WM * SM * 16, BN = WN * SN * 16;
    pol.tiles_x = (rows + BN - 1) / BN;
    const long long tiles = static_cast<long long>(pol.tiles_x) * ((count + BM - 1) / BM);
    if (tiles * split > 0x7fffffffLL || (split > 1 && tiles * (BM * BN / 256) > 0x7fffffffLL))
        return Q3X_HIP_EINVAL;
    if constexpr (HasKSplit<P>::value) {
        if (split > 1 && pol.part == nullptr) return Q3X_HIP_EINVAL;  // the units' sums need a workspace
        pol.ksplit = split;
    } else if (split != 1) {
        return Q3X_HIP_EINVAL;
    }
    hipLaunchKernelGGL((gemm_x3_kernel<QT, WM, WN, SM, SN, P, PF, CF, KS>),
                       dim3(static_cast<unsigned>(tiles * split)), dim3(KS * WM * WN * kWave), 0, stream, pol, rows,
                       cols);
    if constexpr (HasKSplit<P>::value) {
        if (split > 1) {
            const int status = launch_status();
            if (status != Q3X_HIP_OK) return status;
            constexpr int kPerTile = BM * BN / 256;
            hipLaunchKernelGGL((gemm_x3_fixup_kernel<WM, WN, SM, SN, P>),
                               dim3(static_cast<unsigned>(tiles * kPerTile)), dim3(256), 0, stream, pol, rows);
        }
    }
    return launch_status();
}

// A launch by plan; `workspace` bytes at pol.part for split plans
// (policies with a workspace; 0 otherwise).
template <uint32_t QT, class P>
int launch_x3(const P& pol, int rows, int count, int cols, hipStream_t stream, size_t workspace = 0) {
    const X3Plan plan = x3_plan(rows, count, cols, P::kPairedColumns, workspace);
    const int split = plan.split;
    switch (plan.shape) {
        // The one-per-CU shapes with two stages of loads ahead: 1-3% faster
        // than one (and than compute-first) at 512-4096 tokens.
        case X3Shape::k128x256:
            return launch_x3_tiles<QT, 2, 4, 4, 4, 2, false>(pol, rows, count, cols, stream, split);
        case X3Shape::k128x192:
            if constexpr (!P::kPairedColumns)
                return launch_x3_tiles<QT, 2, 4, 4, 3, 2, false>(pol, rows, count, cols, stream, split);
            else
                return launch_x3_tiles<QT, 2, 4, 4, 4, 2, false>(pol, rows, count, cols, stream, split);
        case X3Shape::k64x128_split:
            return launch_x3_tiles<QT, 2, 4, 2, 2, 1, false, P, 2>(pol, rows, count, cols, stream, split);
        case X3Shape::k64x128:
            if (cols >= kX3LongK)
                return launch_x3_tiles<QT, 2, 4, 2, 2, 2, false>(pol, rows, count, cols, stream, split);
            return launch_x3_tiles<QT, 2, 4, 2, 2, 1, false>(pol, rows, count, cols, stream, split);
        default: return launch_x3_tiles<QT, 2, 2, 2, 2, 1, false>(pol, rows, count, cols, stream, split);
    }
}

}  // namespace q3x
