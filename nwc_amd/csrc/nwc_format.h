// nwc_format.h -- format constants and shape arithmetic of NWC v9/v10/v11, shared by the host encoder and the
// gfx950 kernels.  The numbers are fixed by the on-disk format (parda21/NWC csrc/nwc_ops.cu:48-98, docs/format.md
// sections 3, 4b-4d), so they match the reference; the code is this library's own.
#pragma once
#include <cstdint>
#include <hip/hip_runtime.h>

namespace nwc {

constexpr int kVersion = 11;           // nwc_info(0): format 9 = layout 0, 10 = +layout 1 and fp8, 11 = +layout 2
constexpr uint32_t kLanes = 32;        // lane streams per block
constexpr uint32_t kRows0 = 8;         // layout 0 block: 8 rows x 512 columns
constexpr uint32_t kRows12 = 16;       // layouts 1/2 block: 16 rows x 512 columns
constexpr uint32_t kCols = 512;
constexpr uint32_t kBlock = kRows0 * kCols;   // nwc_info(4); the `block` argument must equal it
constexpr uint32_t kHdrBytes = kLanes;        // one header byte per lane and block
constexpr uint32_t kPeek = 12;                // LUT index bits
constexpr uint32_t kLutWords = 1u << kPeek;
// Token-path decode table with a 13-bit window (nwc_seq_table; not part of the format): 2^13 entries already in the
// kernel's step encoding, then exp_of_rank[0..15] packed into four words.
constexpr uint32_t kPeekSeq = 13;
constexpr uint32_t kSeqTableWords = (1u << kPeekSeq) + 4u;
constexpr uint32_t kMaxRankBf16 = 15;         // ranks 0..14 coded r zeros, 1, sign; 15 zeros + 1 = escape
constexpr uint32_t kMaxRankFp8 = 10;          // fp8: 10 symbols, no escape
constexpr uint32_t kFlag = 1u << 30;          // stored-LUT marker of an entry without two complete codes
constexpr uint32_t kNpsym = 1024;             // freq/psym buffer length of the ABI
constexpr uint32_t kRawSlack = 512;           // bytes the Python owner appends to `low`
constexpr int kElemBf16 = 0;
constexpr int kElemFp8 = 1;

__host__ __device__ constexpr int elem_type(int e) { return e & 15; }
__host__ __device__ constexpr int elem_layout(int e) { return (e >> 4) & 15; }
// Layouts 0/1 placed in fixed slots (not a format property; the reference's callers leave bits 8-15 zero): the streams
// of block b start at byte b * stride, so bases[b] = b * stride and `data` holds nb * stride + 128 bytes.  The token
// kernels then compute a block's offset instead of reading it.  Bits 8-15 hold stride / 16; 0 = bases[] only.
__host__ __device__ constexpr uint32_t elem_stride(int e) { return (uint32_t)((e >> 8) & 0xFF) * 16u; }
// Largest stride: a tile's slots plus the 16 bytes read past the last one must fit the smallest region buffer the
// plans give a block (layout 0: 440 words; layout 1: 768 words).
constexpr uint32_t kSlotMax0 = 1728, kSlotMax1 = 3040;
__host__ __device__ constexpr uint32_t slot_max(int layout) {
    return layout == 0 ? kSlotMax0 : layout == 1 ? kSlotMax1 : 0u;
}

// Rounded-up dimensions of an M x K matrix for a layout (nwc_ops.cu:87-98).
struct Shape {
    uint32_t M, K, K16, CB, Mp, nb, rows, nl, nsl, spr, nsl2, spr2;
    __host__ __device__ Shape(uint32_t M_, uint32_t K_, int layout) : M(M_), K(K_) {
        rows = layout ? kRows12 : kRows0;
        K16 = (K + 15u) & ~15u;
        CB = (K + kCols - 1) / kCols;
        Mp = (M + rows - 1) / rows * rows;
        nb = (Mp / rows) * CB;
        nl = (K16 - (CB - 1) * kCols) / 16;          // 16-column chunks coded in the last column block
        nsl = (nl + 1) / 2;                          // its 32-column super-chunks (layouts 1/2)
        spr = 16 * (CB - 1) + nsl;                   // super-chunk slots per 16-row group
        nsl2 = (nsl + 1) / 2;
        spr2 = 8 * (CB - 1) + nsl2;                  // super-chunk pairs per row group (layout 2 fp8 raw plane)
    }
    __host__ __device__ uint32_t groups() const { return Mp / rows; }
    // layout 2: nibble plane [slot][lane][8 B], then the raw plane
    __host__ __device__ uint64_t nib2_bytes() const { return (uint64_t)groups() * spr * kLanes * 8u; }
    __host__ __device__ uint64_t raw2_bytes(int t) const {
        return t == kElemFp8 ? (uint64_t)groups() * spr2 * 3u * kLanes * 4u : (uint64_t)groups() * spr * kLanes * 16u;
    }
    // bytes of `low` without the slack (nwc_ops.cu:111-120)
    __host__ __device__ uint64_t low_bytes(int elem) const {
        const int t = elem_type(elem), lay = elem_layout(elem);
        if (lay == 2) return nib2_bytes() + raw2_bytes(t);
        if (lay) return (uint64_t)groups() * spr * kLanes * (t == kElemFp8 ? 8u : 16u);
        return t == kElemFp8 ? (uint64_t)M * (K16 / 2) : (uint64_t)M * K16;
    }
};

// layouts 1/2 fragment order: lane L = (r = L >> 2, q = L & 3), stream position j (0..15) of a super-chunk
// -> row offset r or r + 8, column offset 8q + 4 (j>>3) + 2 ((j>>2)&1) + (j&1)   (docs/format.md 4c)
__host__ __device__ inline uint32_t frag_row(uint32_t L, uint32_t j) { return (L >> 2) + 8u * ((j >> 1) & 1u); }
__host__ __device__ inline uint32_t frag_col(uint32_t L, uint32_t j) {
    return 8u * (L & 3u) + 4u * ((j >> 3) & 1u) + 2u * ((j >> 2) & 1u) + (j & 1u);
}

}  // namespace nwc
