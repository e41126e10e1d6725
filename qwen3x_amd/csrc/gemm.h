// gemm.h -- FP32-MFMA GEMM with on-the-fly Q8_0 / Q4_0 (or BF16) weight
// conversion (prefill), shared by the dense prefill entry point, the MoE
// grouped GEMM and the MoE layer's router and shared expert.
//
// C[m, n] = sum_k A[m, k] * B[k, n] with A = activations (tokens x cols, FP32,
// row-major) and B = W^T (W = weight rows x cols, quantised).  MFMA's M
// dimension carries tokens and N carries weight rows, so a 32x32 accumulator
// tile stores 32 consecutive output features per token: coalesced writes of
// the row-major [tokens, rows] output.
//
// Per K stage (one 32-column block): the workgroup loads its A tile
// (BM x 32 FP32) and its weight blocks (BN rows x 1 block), converts the
// block values q (Q8_0 int8, Q4_0 nibble - 8) to FP32 and keeps each row's
// fp16 scale d apart, writes both to a double-buffered LDS tile, and each
// wave runs 16 MFMA k-steps per 32x32 tile into a block accumulator that
// starts from zero.  The block's sum then enters the output accumulator as
// acc = fma(d, inner, acc): the reference's per-block factorisation
// (arch/cpu.cpp:64-73, 91-101: inner = sum q * x, sum += d * inner), which
// keeps the rounding error of a K-long sum at the reference's level rather
// than that of one K-long chain of products.  BF16 weights have no block
// scale and accumulate directly.  The 32 k values of a block are fed in the
// order k = 16*(lane/32) + s (s = 0..15), the same permutation for A and B,
// so a lane reads 16 consecutive floats of each operand row with four
// ds_read_b128.
#pragma once

#include <type_traits>
#include <utility>

#include "common.h"

namespace q3x {

constexpr int kGemmPad = 4;            // floats of padding per LDS tile row
constexpr int kXcds = 8;               // MI355X: 8 XCDs of 32 CUs
constexpr int kGemmLd = 32 + kGemmPad; // LDS row pitch (floats), 32x32x2 operand reads
// LDS row pitch of the 16x16x4 operand reads.  Lane group g (lanes 16g ..
// 16g + 15, rows 0..15) reads the 16-byte chunks g and g + 4 of its row:
// with 40-float rows that is conflict-free (measured 112 TB/s of LDS reads
// per GPU, as the 32x32 reads at pitch 36), where the 36-float pitch costs
// 1.44x (70 TB/s).  Two workgroups of 128 x 128 tiles fit one CU's 160 KiB;
// a kernel that also folds per block keeps the block scale of a weight row
// in the row's 8 pad floats rather than in an array of its own.
constexpr int kGemmLd16 = 40;

struct GemmTile {
    int m0;      // first A row of the tile (policy-defined numbering)
    int mcount;  // valid A rows in the tile (<= BM)
    int group;   // policy-defined (expert of a grouped tile)
};

// Raw words of part `part` of PARTS of one block, loaded as whole dwords and
// split only in dequant (after the stage's MFMAs, so the loads stay in
// flight): raw[0] = fp16 scale, raw[1..WORDS] = the part's value bytes.
// Q8_0: elements [part*N, part*N + N), N = 32/PARTS.  Q4_0: nibble bytes
// [NB*part, NB*part + NB), NB = 16/PARTS, i.e. elements NB*part + j (low
// nibbles) and 16 + NB*part + j (high nibbles).  `blk` is 2-byte aligned, so
// the value words are read unaligned.  A part's N values go to the N
// consecutive LDS columns [part*N, part*N + N) (16-byte stores without bank
// conflicts); for Q4_0 that permutes the k order inside a block, and the
// activation tile is stored with the same permutation (a_chunk), so the
// products pair up unchanged.
// BF16 (a router matrix): a "block" is 32 consecutive BF16 values (64 B,
// 4-byte aligned), each word holds two of them and a value is its bits
// shifted up 16 (engine.cpp:181-185), so the conversion is exact.
template <uint32_t QT, int PARTS>
struct BlockPart {
    static constexpr bool kBF16 = QT == Q3X_HIP_MATRIX_BF16;
    static constexpr bool kQ4 = QT == Q3X_HIP_MATRIX_Q4_0;
    static constexpr int N = 32 / PARTS;                                      // elements
    static constexpr int WORDS = (kQ4 ? 16 : kBF16 ? 64 : 32) / PARTS / 4;   // value words
    __device__ static __forceinline__ void load(const uint8_t* blk, int part, uint32_t* raw) {
        if constexpr (kBF16) {
            raw[0] = 0;
            const uint32_t* w = reinterpret_cast<const uint32_t*>(blk);
#pragma unroll
            for (int i = 0; i < WORDS; ++i) raw[1 + i] = w[WORDS * part + i];
        } else {
            raw[0] = *reinterpret_cast<const uint16_t*>(blk);
            __builtin_memcpy(raw + 1, blk + 2 + 4 * WORDS * part, 4 * WORDS);
        }
    }
    // The block values as FP32, out[e] for e < N in the column order of
    // column(): q for Q8_0, nibble - 8 for Q4_0 (the scale is applied per
    // block, scale()), the exact BF16 value for BF16.
    __device__ static __forceinline__ void values(const uint32_t* raw, float* out) {
        if constexpr (kBF16) {
#pragma unroll
            for (int i = 0; i < WORDS; ++i) {
                out[2 * i + 0] = __uint_as_float(raw[1 + i] << 16);
                out[2 * i + 1] = __uint_as_float(raw[1 + i] & 0xffff0000u);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < WORDS; ++i) {
            const uint32_t w = raw[1 + i];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t byte = (w >> (8 * b)) & 0xffu;
                if constexpr (kQ4) {
                    out[4 * i + b] = static_cast<float>(static_cast<int>(byte & 15u) - 8);
                    out[N / 2 + 4 * i + b] = static_cast<float>(static_cast<int>(byte >> 4) - 8);
                } else {
                    out[4 * i + b] = static_cast<float>(static_cast<int8_t>(byte));
                }
            }
        }
    }
    // The block's fp16 scale d (exact in FP32).
    __device__ static __forceinline__ float scale(const uint32_t* raw) { return f16_fast(raw[0]); }
    // Column within the block of output element e.
    __device__ static __forceinline__ int column(int part, int e) { return part * N + e; }
    // LDS chunk (4 columns) of the activations' 16-byte chunk c (elements
    // 4c..4c+3).  Q4_0 with two parts: elements 0-7 | 16-23 | 8-15 | 24-31
    // go to columns 0-7 | 8-15 | 16-23 | 24-31, i.e. chunks 2,3 <-> 4,5.
    __device__ static __forceinline__ int a_chunk(int c) {
        if (QT != Q3X_HIP_MATRIX_Q4_0 || PARTS == 1) return c;
        return (c & 1) | ((c & 2) << 1) | ((c & 4) >> 1);
    }
};

// Policy::kMfma16 (optional, default false): each 32x32 tile is computed as
// 2x2 blocks of 16x16 with v_mfma_f32_16x16x4_f32, so a wave skips the 16-row
// halves that lie past the tile's valid rows (halving the padding work of
// grouped tiles); same MFMA rate as the 32x32x2 form.
template <class P, class = void>
struct Mfma16 { static constexpr bool value = false; };
template <class P>
struct Mfma16<P, decltype(void(P::kMfma16))> { static constexpr bool value = P::kMfma16; };

// Policy::kBlockFold (optional, default true): quantized blocks enter the
// output as acc = fma(d, inner, acc), inner = the block's MFMA sum from zero
// -- the reference's per-block factorisation, which keeps the rounding
// error at the reference's level however long K is.  false: the weight tile
// holds d * q (exact in FP32: an 11-bit scale times a 4- or 8-bit value) and
// one MFMA chain runs over all of K -- about 8% faster on the grouped MoE
// GEMMs, whose K (the hidden size, the expert width) is short.
template <class P, class = void>
struct BlockFold { static constexpr bool value = true; };
template <class P>
struct BlockFold<P, decltype(void(P::kBlockFold))> { static constexpr bool value = P::kBlockFold; };

// Policy::linear_total() (optional, with kLinearGrid): the number of tiles
// of a 1-D grid that is sized for the most tiles possible (a grouped GEMM's
// tile count is known only on the device); workgroups past it return, and
// the XCD remap spreads the live tiles.  Default: the grid size.
template <class P, class = void>
struct LinearTotal {
    __device__ static int get(const P&, int grid) { return grid; }
};
template <class P>
struct LinearTotal<P, decltype(void(std::declval<const P&>().linear_total()))> {
    __device__ static int get(const P& p, int) { return p.linear_total(); }
};

// WM x WN waves, each TM x TN tiles of 32x32.  Policy supplies the tile
// geometry, A rows, weight rows and the output store (see dense / grouped
// policies).  Grid: x = weight-row tiles (BN), y = A-row tiles (BM).
// PF: register sets for the stages ahead (1 or 2): while stage kb computes,
// the loads of stages up to kb + 1 + PF are in flight.
template <uint32_t QT, int WM, int WN, int TM, int TN, class Policy, int PF = 1>
__global__ __launch_bounds__(WM * WN * kWave) void gemm_mfma_kernel(Policy pol, int rows, int cols) {
    static_assert(PF == 1 || PF == 2, "one or two stages in flight");
    constexpr int NT = WM * WN * kWave;   // threads
    constexpr int BM = WM * TM * 32;
    constexpr int BN = WN * TN * 32;
    constexpr int BB = QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : QT == Q3X_HIP_MATRIX_Q4_0 ? kQ4Bytes : kBF16Bytes;
    // A tile load: BM rows x 8 float4 per stage.
    constexpr int A_VEC = BM * 8;
    constexpr int A_PER_T = (A_VEC + NT - 1) / NT;
    // B tile load: BN rows, PARTS threads per row.
    constexpr int PARTS = NT / BN >= 2 ? 2 : 1;
    constexpr int B_ROWS_PER_PASS = NT / PARTS;
    constexpr int B_PASSES = (BN + B_ROWS_PER_PASS - 1) / B_ROWS_PER_PASS;
    constexpr int PER_PART = 32 / PARTS;
    static_assert(PARTS * B_ROWS_PER_PASS == NT, "thread split");

    constexpr bool M16 = Mfma16<Policy>::value;
    constexpr int LD = M16 ? kGemmLd16 : kGemmLd;
    // Block scales of the stage's weight rows (quantized types): their own
    // array, or (16x16 layout) float 32 of the weight row's padding.
    constexpr bool kScaled = QT != Q3X_HIP_MATRIX_BF16;
    constexpr bool kFold = kScaled && BlockFold<Policy>::value;
    constexpr int A_FLOATS = BM * LD, B_FLOATS = BN * LD, D_FLOATS = kFold && !M16 ? BN : 0;
    __shared__ __attribute__((aligned(16))) float lds_tiles[2 * (A_FLOATS + B_FLOATS + D_FLOATS)];
    auto As = [&](int buf) { return lds_tiles + buf * A_FLOATS; };
    auto Bs = [&](int buf) { return lds_tiles + 2 * A_FLOATS + buf * B_FLOATS; };
    auto Ds = [&](int buf, int n) -> float& {
        if constexpr (M16) return lds_tiles[2 * A_FLOATS + buf * B_FLOATS + n * LD + 32];
        else return lds_tiles[2 * (A_FLOATS + B_FLOATS) + buf * BN + n];
    };

    // Tile coordinates: a 2-D grid (x = weight-row tiles, y = A-row tiles), or
    // a 1-D grid over gx * gy tiles (Policy::kLinearGrid) remapped so that
    // each XCD (workgroups are dealt to the 8 XCDs round-robin) takes a
    // contiguous run of tiles: workgroups that share an A tile (same y,
    // consecutive x) then share one XCD's L2.
    int bx = blockIdx.x, by = blockIdx.y;
    if constexpr (Policy::kLinearGrid) {
        const int total = LinearTotal<Policy>::get(pol, gridDim.x), L = blockIdx.x;
        if (L >= total) return;
        const int q = total / kXcds, r = total % kXcds, xcd = L % kXcds, k = L / kXcds;
        const int t = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + k;
        bx = t % pol.tiles_x;
        by = t / pol.tiles_x;
    }
    GemmTile tile;
    if (!pol.tile(by, BM, tile)) return;
    const int n0 = bx * BN;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int wm = wave / WN, wn = wave % WN;
    const int li = lane & 31, kh = lane >> 5;

    // Per-thread source pointers, fixed over K.  Every thread loads every
    // stage, with no branch, so the compiler counts the loads in flight
    // exactly (a load under a lane-dependent branch makes it wait for all of
    // them): rows past the tile's valid A rows, past the matrix's weight rows
    // or past the tile (threads with no row of their own) read a valid row
    // instead.  An output row depends only on its own A row, a column only
    // on its own weight row, and those outputs are never stored; the extra
    // rows are not written to LDS either.
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

    using Part = BlockPart<QT, PARTS>;
    f32x4 a_reg[PF][A_PER_T];
    uint32_t b_raw[PF][B_PASSES][1 + Part::WORDS];
    auto load_stage = [&](int kb, int r) {
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) a_reg[r][i] = *reinterpret_cast<const f32x4*>(a_src[i] + 32 * kb);
#pragma unroll
        for (int p = 0; p < B_PASSES; ++p) Part::load(b_src[p] + static_cast<size_t>(kb) * BB, b_part, b_raw[r][p]);
    };
    auto store_stage = [&](int buf, int r) {
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            const int idx = tid + i * NT;
            if (idx < A_VEC)
                *reinterpret_cast<f32x4*>(&As(buf)[(idx >> 3) * LD + 4 * Part::a_chunk(idx & 7)]) = a_reg[r][i];
        }
#pragma unroll
        for (int p = 0; p < B_PASSES; ++p) {
            const int n = tid / PARTS + p * B_ROWS_PER_PASS;
            if (n < BN) {
                float vals[PER_PART];
                Part::values(b_raw[r][p], vals);
                if constexpr (kFold) {
                    if (b_part == 0) Ds(buf, n) = Part::scale(b_raw[r][p]);
                } else if constexpr (kScaled) {
                    const float d = Part::scale(b_raw[r][p]);
#pragma unroll
                    for (int e = 0; e < PER_PART; ++e) vals[e] *= d;  // exact
                }
#pragma unroll
                for (int e = 0; e < PER_PART; e += 4) {
                    const int c = Part::column(b_part, e);
                    *reinterpret_cast<f32x4*>(&Bs(buf)[n * LD + c]) =
                        f32x4{vals[e], vals[e + 1], vals[e + 2], vals[e + 3]};
                }
            }
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    // 16x16 form: acc16[q][j][nh] is block (rows 16q.., cols nh*16..) of the
    // wave's 32-row tile q / 2, column tile j: subtile q = 2 i + mh holds rows
    // (wm * TM + i) * 32 + mh * 16 + [0, 16); lane l holds rows 4*(l/16) + r,
    // column l % 16.
    constexpr int NSUB = 2 * TM;
    f32x4 acc16[NSUB][TN][2];
#pragma unroll
    for (int q = 0; q < NSUB; ++q)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int nh = 0; nh < 2; ++nh) acc16[q][j][nh] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int l16 = lane & 15, g16 = lane >> 4;

    const int nblk = cols / kBlock;
    // A wave whose A rows all lie past the tile's valid rows (the last tile
    // of an expert's group) has nothing to compute: it only helps stage the
    // tiles, leaving the SIMD's matrix core to the other waves.  Its active
    // 16-row subtiles form a prefix of the subtile order.
    const bool active = !Policy::kPartialTiles || wm * TM * 32 < tile.mcount;
    const int nsub = Policy::kPartialTiles ? min(NSUB, (tile.mcount - wm * TM * 32 + 15) / 16) : NSUB;

    // Quantized types: each tile's MFMA chain sums one block into a block
    // accumulator from zero, and the block enters acc as acc = fma(d, inner,
    // acc), blocks in order.  A tile's fold is issued after the next tile's
    // MFMA chain, so the matrix core runs while the VALU folds; the last
    // tile of a stage is folded in the next stage, right after its first
    // chain (or after the loop), with the scales of its own stage kept in
    // registers (the next stage's staging overwrites them in LDS).  A wave
    // with one 32x32 tile alternates two block accumulators between stages.
    constexpr int NT32 = TM * TN;
    constexpr int SETS = NT32 == 1 ? 2 : 1;
    f32x16 blk[SETS][NT32];
    float d_old[TN], d_new[TN];
    f32x4 blk16[NSUB][TN][2];
    float d16_old[TN][2], d16_new[TN][2];
    auto fold32 = [&](int t, const f32x16& b, const float* d) {
        const int i = t / TN, j = t % TN;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(d[j], b[r], acc[i][j][r]);
    };
    auto fold16 = [&](int q, float (*d)[2]) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int nh = 0; nh < 2; ++nh)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc16[q][j][nh][r] = fmaf(d[j][nh], blk16[q][j][nh][r], acc16[q][j][nh][r]);
    };
    // The pending subtile of the previous stage (the last active one).
    auto fold16_pending = [&]() {
#pragma unroll
        for (int q = 0; q < NSUB; ++q)
            if (q == nsub - 1) fold16(q, d16_old);
    };

    // One K stage kb: first stage kb + 1 (in registers since the previous
    // stage) goes to the other LDS buffer, which the previous barrier freed;
    // then the loads of stage kb + 1 + PF are issued into the register set
    // just emptied; then the MFMAs of stage kb; then the barrier.  At the LDS
    // store the only loads in flight are the ones it consumes (so the
    // compiler waits for exactly those), and the new loads overlap a whole
    // stage of MFMAs and the barrier.  Stage s lives in register set s % PF;
    // P is the stage's parity (the block accumulator set of one-tile waves).
    auto step = [&](int kb, int r, auto parity) {
        constexpr int P = decltype(parity)::value;
        const int buf = kb & 1;
        if (kb + 1 < nblk) store_stage(buf ^ 1, r);
        if (kb + 1 + PF < nblk) load_stage(kb + 1 + PF, r);
        if (M16 && active) {
            // Lane group g16 supplies, at MFMA step s, k = 4 * g16 + s for s < 4
            // and k = 16 + 4 * g16 + (s - 4) after (the same k order for both
            // operands): the 16-byte chunks g16 and g16 + 4 of the row.
            f32x4 bf[TN][2][2];
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int nh = 0; nh < 2; ++nh) {
                    const float* src = &Bs(buf)[((wn * TN + j) * 32 + nh * 16 + l16) * LD + 4 * g16];
                    bf[j][nh][0] = *reinterpret_cast<const f32x4*>(src);
                    bf[j][nh][1] = *reinterpret_cast<const f32x4*>(src + 16);
                }
            if constexpr (kFold) {
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int nh = 0; nh < 2; ++nh) d16_new[j][nh] = Ds(buf, (wn * TN + j) * 32 + nh * 16 + l16);
                // One active subtile: its pending block is folded before the
                // chain reuses its accumulator.
                if (kb > 0 && nsub == 1) fold16_pending();
            }
#pragma unroll
            for (int q = 0; q < NSUB; ++q) {
                if (q >= nsub) break;
                const float* asrc = &As(buf)[((wm * TM + q / 2) * 32 + (q & 1) * 16 + l16) * LD + 4 * g16];
                const f32x4 af0 = *reinterpret_cast<const f32x4*>(asrc);
                const f32x4 af1 = *reinterpret_cast<const f32x4*>(asrc + 16);
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    const float a = s < 4 ? af0[s] : af1[s - 4];
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int nh = 0; nh < 2; ++nh) {
                            const float b = bf[j][nh][s >> 2][s & 3];
                            if constexpr (kFold)
                                blk16[q][j][nh] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                                    a, b, s == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : blk16[q][j][nh], 0, 0, 0);
                            else
                                acc16[q][j][nh] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc16[q][j][nh], 0, 0, 0);
                        }
                }
                if constexpr (kFold) {
                    if (q == 0 && kb > 0 && nsub > 1) fold16_pending();
                    if (q > 0) fold16(q - 1, d16_new);
                }
            }
            if constexpr (kFold) {
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int nh = 0; nh < 2; ++nh) d16_old[j][nh] = d16_new[j][nh];
            }
        } else if (active) {
            f32x4 af[TM][4], bf[TN][4];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const float* src = &As(buf)[((wm * TM + i) * 32 + li) * LD + 16 * kh];
#pragma unroll
                for (int q = 0; q < 4; ++q) af[i][q] = *reinterpret_cast<const f32x4*>(src + 4 * q);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const float* src = &Bs(buf)[((wn * TN + j) * 32 + li) * LD + 16 * kh];
#pragma unroll
                for (int q = 0; q < 4; ++q) bf[j][q] = *reinterpret_cast<const f32x4*>(src + 4 * q);
            }
            if constexpr (kFold) {
#pragma unroll
                for (int j = 0; j < TN; ++j) d_new[j] = Ds(buf, (wn * TN + j) * 32 + li);
                constexpr int S = P % SETS;
#pragma unroll
                for (int t = 0; t < NT32; ++t) {
                    const int i = t / TN, j = t % TN;
#pragma unroll
                    for (int s = 0; s < 16; ++s)
                        blk[S][t] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s >> 2][s & 3], bf[j][s >> 2][s & 3],
                                                                         s == 0 ? f32x16{} : blk[S][t], 0, 0, 0);
                    if (t == 0 && kb > 0) {
                        // The previous stage's last tile: in the other set
                        // for one-tile waves, else the last tile of this set.
                        if constexpr (SETS == 2) fold32(0, blk[S ^ 1][0], d_old);
                        else fold32(NT32 - 1, blk[0][NT32 - 1], d_old);
                    }
                    if (t > 0) fold32(t - 1, blk[S][t - 1], d_new);
                }
#pragma unroll
                for (int j = 0; j < TN; ++j) d_old[j] = d_new[j];
            } else {
#pragma unroll
                for (int s = 0; s < 16; ++s)
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s >> 2][s & 3],
                                                                             bf[j][s >> 2][s & 3],
                                                                             acc[i][j], 0, 0, 0);
            }
        }
        __syncthreads();
    };
    // Prologue: stage 0 into LDS buffer 0, stages 1..PF into registers.
    load_stage(0, 0);
    store_stage(0, 0);
#pragma unroll
    for (int q = 1; q <= PF; ++q)
        if (q < nblk) load_stage(q, q % PF);
    __syncthreads();
    // Stages in pairs, so each knows its parity at compile time.
    for (int kb = 0; kb < nblk; kb += 2) {
        step(kb, PF == 1 ? 0 : 1, std::integral_constant<int, 0>{});         // PF 2: stage kb + 1 is in set 1
        if (kb + 1 < nblk) step(kb + 1, 0, std::integral_constant<int, 1>{});  // PF 2: stage kb + 2 is in set 0
    }
    // The last stage's pending tile.
    if (kFold && active) {
        if constexpr (M16) {
            fold16_pending();
        } else if constexpr (SETS == 2) {
            if ((nblk - 1) & 1) fold32(0, blk[1][0], d_old);
            else fold32(0, blk[0][0], d_old);
        } else {
            fold32(NT32 - 1, blk[0][NT32 - 1], d_old);
        }
    }
    if constexpr (M16) {
        // v_mfma_f32_16x16x4_f32: register r of lane l holds C[4*(l/16) + r][l%16].
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int mh = 0; mh < 2; ++mh)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int nb = n0 + (wn * TN + j) * 32 + l16;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int m = (wm * TM + i) * 32 + mh * 16 + 4 * g16 + r;
                        if (m >= tile.mcount) continue;
                        if constexpr (Policy::kPairedColumns) {
                            // Column q < 16 and its partner q + 16 sit in the
                            // same lane: blocks nh = 0 and nh = 1.
                            if (nb < rows) pol.store_pair(tile, m, nb, acc16[2 * i + mh][j][0][r], acc16[2 * i + mh][j][1][r]);
                        } else {
#pragma unroll
                            for (int nh = 0; nh < 2; ++nh)
                                if (nb + 16 * nh < rows) pol.store(tile, m, nb + 16 * nh, acc16[2 * i + mh][j][nh][r]);
                        }
                    }
                }
        return;
    }
    // Accumulator layout of v_mfma_f32_32x32x2f32: register r of lane l holds
    // C[8*(r/4) + 4*(l/32) + r%4][l%32].
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + (wn * TN + j) * 32 + li;
            if constexpr (Policy::kPairedColumns) {
                // Columns li and li + 16 of a 32-column tile form a pair
                // (e.g. gate and up of one output feature): lane li < 16
                // receives its partner's value and stores the pair.
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float partner = __shfl_xor(acc[i][j][r], 16);
                    const int m = (wm * TM + i) * 32 + 8 * (r >> 2) + 4 * kh + (r & 3);
                    if (!(li & 16) && n < rows && m < tile.mcount) pol.store_pair(tile, m, n, acc[i][j][r], partner);
                }
            } else {
                if (n >= rows) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = (wm * TM + i) * 32 + 8 * (r >> 2) + 4 * kh + (r & 3);
                    if (m < tile.mcount) pol.store(tile, m, n, acc[i][j][r]);
                }
            }
        }
}

}  // namespace q3x
