// gemm.h -- shared pieces of the prefill GEMMs (gemm_x3.h): the tile a
// policy hands the kernel, the raw load and conversion of a weight block's
// values, and the 1-D grid's tile count.
//
// C[m, n] = sum_k A[m, k] * B[k, n] with A = activations (tokens x cols, FP32,
// row-major) and B = W^T (W = weight rows x cols, quantised).  The matrix
// instructions' M dimension carries A rows and N carries weight rows, so an
// output block stores consecutive output features per token: coalesced
// writes of the row-major [tokens, rows] output.
#pragma once

#include <type_traits>
#include <utility>

#include "common.h"

namespace q3x {

constexpr int kXcds = 8;  // MI355X: 8 XCDs of 32 CUs

struct GemmTile {
    int m0;      // first A row of the tile (policy-defined numbering)
    int mcount;  // valid A rows in the tile (<= BM)
    int group;   // policy-defined (expert of a grouped tile)
};

// Raw words of part `part` of PARTS of one block, loaded as whole dwords and
// split only when the stage is written to LDS (a stage later, so the loads
// stay in flight): raw[0] = fp16 scale, raw[1..WORDS] = the part's value
// bytes.
// Q8_0: elements [part*N, part*N + N), N = 32/PARTS.  Q4_0: nibble bytes
// [NB*part, NB*part + NB), NB = 16/PARTS, i.e. elements NB*part + j (low
// nibbles) and 16 + NB*part + j (high nibbles).  `blk` is 2-byte aligned, so
// the value words are read unaligned.  A part's N values go to the N
// consecutive LDS columns [part*N, part*N + N); for Q4_0 that permutes the
// k order inside a block, and the activation tile is stored with the same
// permutation, so the products pair up unchanged.
// BF16 (a router matrix): a "block" is 32 consecutive BF16 values (64 B,
// 4-byte aligned), each word holds two of them and a value is its bits
// shifted up 16 (engine.cpp:181-185), so the conversion is exact.
template <uint32_t QT, int PARTS>
struct BlockPart {
    static constexpr bool kBF16 = QT == Q3X_HIP_MATRIX_BF16;
    static constexpr bool kQ4 = QT == Q3X_HIP_MATRIX_Q4_0;
    static constexpr int N = 32 / PARTS;                                      // elements
    static constexpr int WORDS = (kQ4 ? 16 : kBF16 ? 64 : 32) / PARTS / 4;   // value words
    // Q4_0 in two parts: one 12-byte load a part (part 0 block bytes 0-11,
    // part 1 bytes 6-17), where two loads (the scale, then the part's 8
    // value bytes) would each take an address slot of the vector memory
    // pipeline; finish() puts the words in place when the stage is
    // converted, part 1 taking the scale from its row's other lane.
    static constexpr bool kOneLoad = kQ4 && PARTS == 2;
    __device__ static __forceinline__ void load(const uint8_t* blk, int part, uint32_t* raw) {
        if constexpr (kOneLoad) {
            __builtin_memcpy(raw, blk + 6 * part, 12);
        } else if constexpr (kBF16) {
            raw[0] = 0;
            const uint32_t* w = reinterpret_cast<const uint32_t*>(blk);
#pragma unroll
            for (int i = 0; i < WORDS; ++i) raw[1 + i] = w[WORDS * part + i];
        } else {
            raw[0] = *reinterpret_cast<const uint16_t*>(blk);
            __builtin_memcpy(raw + 1, blk + 2 + 4 * WORDS * part, 4 * WORDS);
        }
    }
    // raw as load() leaves it -> [scale, value words]; every lane of the
    // wave active (the two parts of a row are lanes 2k and 2k + 1).
    __device__ static __forceinline__ void finish(uint32_t* raw, int part) {
        if constexpr (kOneLoad) {
            const uint32_t partner = dpp_u32<0xB1>(raw[0]);  // lane ^ 1: part 0's bytes 0-3
            const uint32_t scale = (part ? partner : raw[0]) & 0xffffu;
            const uint32_t w0 = part ? raw[1] : __builtin_amdgcn_alignbyte(raw[1], raw[0], 2);
            const uint32_t w1 = part ? raw[2] : __builtin_amdgcn_alignbyte(raw[2], raw[1], 2);
            raw[0] = scale;
            raw[1] = w0;
            raw[2] = w1;
        }
    }
    // The block values as FP32, out[e] for e < N in the LDS column order
    // (column part*N + e): q for Q8_0, 16 (nibble - 8) for Q4_0 (the scale
    // is applied per block, scale()), the exact BF16 value for BF16.
    // Q4_0: a nibble n moved to the top of its byte with bit 3 flipped,
    // ((n ^ 8) << 4), is the signed byte 16 (n - 8), so one xor-and per four
    // values gives bytes that convert as signed bytes; the factor 16 is a
    // power of two, exact in every product and sum, and scale() returns d / 16.
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
            if constexpr (kQ4) {
                const uint32_t lo = ((w << 4) ^ 0x80808080u) & 0xf0f0f0f0u;  // low nibbles
                const uint32_t hi = (w ^ 0x80808080u) & 0xf0f0f0f0u;         // high nibbles
                out[4 * i + 0] = sbyte<0>(lo);
                out[4 * i + 1] = sbyte<1>(lo);
                out[4 * i + 2] = sbyte<2>(lo);
                out[4 * i + 3] = sbyte<3>(lo);
                out[N / 2 + 4 * i + 0] = sbyte<0>(hi);
                out[N / 2 + 4 * i + 1] = sbyte<1>(hi);
                out[N / 2 + 4 * i + 2] = sbyte<2>(hi);
                out[N / 2 + 4 * i + 3] = sbyte<3>(hi);
            } else {
                out[4 * i + 0] = sbyte<0>(w);
                out[4 * i + 1] = sbyte<1>(w);
                out[4 * i + 2] = sbyte<2>(w);
                out[4 * i + 3] = sbyte<3>(w);
            }
        }
    }
    // The block's fp16 scale d (exact in FP32); d / 16 for Q4_0, whose
    // values() are 16 (n - 8).
    __device__ static __forceinline__ float scale(const uint32_t* raw) {
        return kQ4 ? f16_fast(raw[0]) * 0.0625f : f16_fast(raw[0]);
    }
};

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

}  // namespace q3x
