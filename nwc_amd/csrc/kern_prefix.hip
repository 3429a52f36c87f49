// kern_prefix.hip -- gfx950 kernels for the prefix-coded layouts 0 (8 x 512 blocks, row-major lanes; format v9) and
// 1 (16 x 512 blocks in tensor-core fragment order; format v10), BF16 and fp8.
//
// Work decomposition: a workgroup owns G whole row groups (all CB column blocks of them); each 32-lane half-wave
// decodes one block at a time, keeps the partial row sums of the block in LDS, and the workgroup finishes its
// rows itself (sum over column blocks, scale, bias, BF16 rounding).  The reference needs a second kernel and a
// global scratch buffer for that step (nwc_ops.cu:553-565, :1139).
//
// Memory: a half-wave first copies its block's 32 lane streams into an LDS slot with 16-byte loads and requests all
// of its raw-plane rows, with one wait per block; the decode loop then issues no global loads (every refill of the
// bit window is a ds_read).
//
// Inner loop per lane: four codes per window step (two table reads, one funnel-shift advance, at most one
// refill), one v_perm_b32 per weight pair to assemble [raw | exponent] BF16 pairs, one v_dot2_f32_bf16 per pair
// against BF16 activations in registers (fp32 activations: two v_perm_b32 + two FMAs per pair).
#include "nwc_device.h"
#include "nwc_launch.h"

namespace nwc {

// Activations of a lane: 16 columns as 8 BF16 pairs, or 16 fp32 values.
template <bool XBF16> struct XRegs;
template <> struct XRegs<true> { uint32_t b[8]; };
template <> struct XRegs<false> { float f[16]; };

// ---------------------------------------------------------------------------------------------------------------
// Layout 0: lane L of block (rb, cb) owns columns cb*512 + 16L .. +15 of rows rb*8 .. rb*8+7, stream order row-major.
// Raw-plane row of a lane (16 weights: word k holds weights 4k..4k+3).  Loads are unconditional and unmasked, so a
// loop that issues them keeps static wait counts and no select waits for the data: rows past M read row M - 1, and
// columns past K16 read into the next row (or the 512 slack bytes after the plane).  Those products are garbage and
// are dropped: sums of lanes past K16 are zeroed (col_ok selects), rows past M are never stored.
template <int ELEM>
__device__ __forceinline__ uint4 raw_row0(const uint8_t *__restrict__ low, const Shape &f, uint32_t row, uint32_t col0, bool col_ok) {
    const bool ok = row < f.M && col_ok;
    const uint32_t r = ok ? row : 0u, c = ok ? col0 : 0u;
    if (ELEM == kElemFp8) return expand_nibbles(ldnt2(low + (r * (f.K16 / 2) + c / 2)));
    return ldnt4(low + (r * f.K16 + c));
}

template <bool XBF16>
__device__ __forceinline__ void load_x16(XRegs<XBF16> &x, const void *xp, uint32_t col0, bool col_ok) {
    const uint32_t c = col_ok ? col0 : 0u;
    if constexpr (XBF16) {
        const uint4 *p = (const uint4 *)((const uint16_t *)xp + c);
        const uint4 v0 = p[0], v1 = p[1];
        x.b[0] = v0.x; x.b[1] = v0.y; x.b[2] = v0.z; x.b[3] = v0.w; x.b[4] = v1.x; x.b[5] = v1.y; x.b[6] = v1.z; x.b[7] = v1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = ((const float4 *)((const float *)xp + c))[i];
            x.f[4 * i] = v.x; x.f[4 * i + 1] = v.y; x.f[4 * i + 2] = v.z; x.f[4 * i + 3] = v.w;
        }
    }
}

// Position of block t (0 <= t < G * CB) of a workgroup's tile for lane L.
struct Coord0 {
    uint32_t g, cb, b, row0, col0;
    uint32_t rb, rmax;          // raw-plane byte offsets of (row0, col0) and (M - 1, col0)
    bool col_ok;
};
__device__ __forceinline__ Coord0 coord0(uint32_t t, uint32_t rg0, const Shape &f, uint32_t L) {
    Coord0 c;
    c.g = t / f.CB;
    c.cb = t - c.g * f.CB;
    const uint32_t rb = rg0 + c.g;
    c.b = rb * f.CB + c.cb;
    c.row0 = rb * kRows0;
    c.col0 = c.cb * kCols + L * 16;
    c.col_ok = c.col0 < f.K16;
    c.rb = c.row0 * f.K16 + c.col0;                          // BF16: one byte per weight; fp8: halved below
    c.rmax = (f.M - 1u) * f.K16 + c.col0;
    return c;
}

// Raw-plane row r of block c (see raw_row0 for the out-of-range rules); the row offset r * stride is uniform.
template <int ELEM>
__device__ __forceinline__ uint4 raw_row(const uint8_t *__restrict__ low, const Shape &f, const Coord0 &c, uint32_t r) {
    const uint32_t off = min(c.rb + r * f.K16, c.rmax);
    if (ELEM == kElemFp8) return expand_nibbles(ldnt2(low + off / 2));
    return ldnt4(low + off);
}

// Bit position where part j (0-3) of block b starts in lane L's stream: 0 for the first part, else row-index entry
// j - 1.  The entry is loaded for every part (the first part's load reads entry 0 and drops it): a load inside a branch
// makes the compiler wait at the branch's end for it and for every request before it, which would hold back the
// stream copy by a whole round trip.  Callers request it after their other prologue loads (the compiler may read its
// register as the don't-care high half of a 64-bit multiply-add operand, which would wait for it).
__device__ __forceinline__ uint32_t part_start(const BlockArgs &a, uint32_t b, uint32_t j, uint32_t L) {
    const uint32_t v = a.aux[((uint64_t)b * kRowIndexSplits + (j ? j - 1u : 0u)) * kLanes + L];
    return j ? v : 0u;
}

// Weights of one window step for the accumulator / dequant output.
template <int MODE, bool XBF16>
__device__ __forceinline__ void use_quad(uint32_t e1, uint32_t e2, uint32_t rk, int k, const XRegs<XBF16> &x, float &sum,
                                         uint32_t pw[8]) {
    if constexpr (MODE == kRowIndex) {
        (void)e1; (void)e2; (void)rk; (void)k; (void)x; (void)sum; (void)pw;
    } else if constexpr (MODE == kDequant) {
        pw[2 * k] = perm(e1, rk, kSelPair0);
        pw[2 * k + 1] = perm(e2, rk, kSelPair2);
    } else if constexpr (XBF16) {
        sum = dot2_bf16(perm(e1, rk, kSelPair0), x.b[2 * k], sum);
        sum = dot2_bf16(perm(e2, rk, kSelPair2), x.b[2 * k + 1], sum);
    } else {
        sum = fmaf(__uint_as_float(perm(e1, rk, sel_f32(0, 5))), x.f[4 * k], sum);
        sum = fmaf(__uint_as_float(perm(e1, rk, sel_f32(1, 6))), x.f[4 * k + 1], sum);
        sum = fmaf(__uint_as_float(perm(e2, rk, sel_f32(2, 5))), x.f[4 * k + 2], sum);
        sum = fmaf(__uint_as_float(perm(e2, rk, sel_f32(3, 6))), x.f[4 * k + 3], sum);
    }
}

template <int MODE>
__device__ __forceinline__ void store_row0(const BlockArgs &a, const Shape &f, uint32_t row, uint32_t col0, bool col_ok,
                                           const uint32_t pw[8]) {
    if (row < f.M && col_ok) {
        uint4 *o = (uint4 *)((uint16_t *)a.out + (uint64_t)row * f.K16 + col0);
        o[0] = make_uint4(pw[0], pw[1], pw[2], pw[3]);
        o[1] = make_uint4(pw[4], pw[5], pw[6], pw[7]);
    }
}

// ---- workgroup staging of the streams of a run of consecutive blocks ----
// The blocks of a workgroup's tile are consecutive in `data`, so a round of H blocks (one per half-wave) is one
// contiguous byte range: [bases[b_lo], bases[b_hi]) -- for the matrix's last block, its base plus four bytes per header
// word.  All threads copy it into LDS with 16-byte loads; no half-wave needs its own header scan before the copy.
// With fixed slots (stride != 0) the range is [b_lo * stride, b_hi * stride) and nothing is read to find it.
struct Region {
    uint32_t lo16, n16;         // 16-byte aligned start (byte offset into data), 16-byte chunks
};

// One past the last stream byte of the matrix (block nb - 1: its base plus four bytes per header word).
__device__ __forceinline__ uint32_t matrix_end(const BlockArgs &a, uint32_t nb) {
    const uint32_t *h = (const uint32_t *)(a.hdr + (uint64_t)(nb - 1u) * kHdrBytes);
    uint32_t words = 0;
#pragma unroll
    for (int i = 0; i < (int)kHdrBytes / 4; i++) words = __builtin_amdgcn_udot4(h[i], 0x01010101u, words, false);
    return a.bases[nb - 1u] + 4u * words;
}

// Blocks [b_lo, b_hi) plus the 16 bytes the last lane's window reads past its stream (inside the 64 slack bytes that
// follow the matrix's last block, or the 128 after its last slot).  stride: a.stride (fixed slots) or 0 (bases[]).
__device__ __forceinline__ Region region_of(const BlockArgs &a, uint32_t b_lo, uint32_t b_hi, uint32_t nb, uint32_t mend,
                                            uint32_t stride) {
    Region r;
    if (stride) {
        r.lo16 = b_lo * stride;                                 // a multiple of 16
        r.n16 = ((b_hi > b_lo ? b_hi - b_lo : 0u) * stride + 31u) >> 4;
        return r;
    }
    const uint32_t s = a.bases[b_lo], e = a.bases[min(b_hi, nb - 1u)];
    r.lo16 = s & ~15u;
    r.n16 = ((b_hi < nb ? e : mend) + 16u - r.lo16 + 15u) >> 4;
    return r;
}

// Four 16-byte chunks per thread cover a region buffer of up to 512 words per half-wave; native vectors keep the
// words in registers.  Only chunks inside the region are requested (a wave wholly past it issues nothing): the
// prologue's vector-memory instructions all pass through the CU's address unit, so a workgroup that requested its
// full four chunks per thread would delay the other workgroup on its CU (o_proj: 9.3 -> 8.7 us).
struct Bulk {
    u32x4_t v0, v1, v2, v3;
};
__device__ __forceinline__ void bulk_issue(Bulk &B, const uint8_t *__restrict__ data, const Region &r, uint32_t tid, uint32_t nth) {
    const uint8_t *p = data + r.lo16;
    if (tid < r.n16) B.v0 = *(const u32x4_t *)(p + 16u * tid);
    if (tid + nth < r.n16) B.v1 = *(const u32x4_t *)(p + 16u * (tid + nth));
    if (tid + 2u * nth < r.n16) B.v2 = *(const u32x4_t *)(p + 16u * (tid + 2u * nth));
    if (tid + 3u * nth < r.n16) B.v3 = *(const u32x4_t *)(p + 16u * (tid + 3u * nth));
}
__device__ __forceinline__ void bulk_commit(const Bulk &B, uint32_t *buf, const Region &r, uint32_t tid, uint32_t nth) {
    if (tid < r.n16) *(u32x4_t *)(buf + 4u * tid) = B.v0;
    if (tid + nth < r.n16) *(u32x4_t *)(buf + 4u * (tid + nth)) = B.v1;
    if (tid + 2u * nth < r.n16) *(u32x4_t *)(buf + 4u * (tid + 2u * nth)) = B.v2;
    if (tid + 3u * nth < r.n16) *(u32x4_t *)(buf + 4u * (tid + 3u * nth)) = B.v3;
}

// One row of a layout-0 block for one lane (16 weights = four steps of the cursor), dot product with the lane's
// activations or, for dequantization, the eight BF16 pairs in pw.  A step whose table entries were not both fast in
// some lane of the wave is redone code by code from its start by the whole wave (0.09% of lane-steps, 5% of
// wave-steps for N(0, 0.02^2) BF16 at a 12-bit window).
template <int ELEM, int MODE, bool XBF16, int STRIDE = 1, class Tab>
__device__ __forceinline__ float row0(Seq<ELEM, STRIDE> &S, const Tab &s, const uint4 &rw, const XRegs<XBF16> &x,
                                      uint32_t pw[8]) {
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t s0 = S.s;
        const uint32_t *wp0 = S.wp;
        uint32_t e1, e2;
        if (__builtin_expect(__any(S.fast_quad(s, e1, e2) >= kSeqSlowTest), 0)) {
            S.s = s0;
            S.wp = wp0;
            S.reload();
            S.slow_quad(s, e1, e2);
        }
        use_quad<MODE, XBF16>(e1, e2, u4_get(rw, k), k, x, sum, pw);
        // consume each step's weights before the next decode step (otherwise the compiler sinks every dot product to
        // the end of the unrolled block and keeps all decoded words live)
        if (MODE == kDequant) asm volatile("" : "+v"(pw[2 * k]), "+v"(pw[2 * k + 1]));
        else if (MODE != kRowIndex) asm volatile("" : "+v"(sum));
    }
    return sum;
}

// Raw rows in flight per half-wave: two.  The prologue requests rows 0-1 only once the wave's stream chunks have
// arrived, so decoding starts sooner (a deeper ring, or rows requested together with the streams, measured slower:
// the whole chip's first requests compete for HBM, and the workgroup waits for all of its streams).
constexpr int kRing0 = 2;
// Dequantization requests all of a half-wave's raw rows at once: its row stores share the in-order vector-memory
// counter with the raw loads, so a wait for raw row r also waits for every store requested before row r's load (4B
// dequantization per stack, ring of 2 / 4 / 8 rows: 3072 / 3047 / 2929 us; gate_up 38.8 / 37.8 / 35.2 us).
constexpr int kRingD = 8;
template <int MODE>
constexpr int ring_depth() { return MODE == kDequant ? kRingD : kRing0; }

// The table entries of one row's 16 weights for one lane (four steps of the cursor; a step that was not fast in some
// lane is redone code by code by the whole wave), kept apart from their use so that a row can be decoded before its
// raw bytes have arrived.
template <int ELEM, class Tab>
__device__ __forceinline__ void row_codes(Seq<ELEM> &S, const Tab &s, uint32_t (&e1)[4], uint32_t (&e2)[4]) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t s0 = S.s;
        const uint32_t *wp0 = S.wp;
        if (__builtin_expect(__any(S.fast_quad(s, e1[k], e2[k]) >= kSeqSlowTest), 0)) {
            S.s = s0;
            S.wp = wp0;
            S.reload();
            S.slow_quad(s, e1[k], e2[k]);
        }
    }
}
// The lane's partial dot product of one row from its entries, raw bytes and activations (token and fp32 modes).
template <int MODE, bool XBF16>
__device__ __forceinline__ float row_dot(const uint32_t (&e1)[4], const uint32_t (&e2)[4], const uint4 &rw,
                                         const XRegs<XBF16> &x) {
    float sum = 0.f;
    uint32_t pw[8];
#pragma unroll
    for (int k = 0; k < 4; k++) use_quad<MODE, XBF16>(e1[k], e2[k], u4_get(rw, k), k, x, sum, pw);
    asm volatile("" : "+v"(sum));                            // one row's products before the next row's
    return sum;
}

// Rows r0 .. r0 + NR - 1 of one layout-0 block for one lane, decoded from LDS starting at bit position P0 of the
// lane's stream, with the first kRing0 of those raw-plane rows already requested into `ring` (c.rb is row r0's
// offset).  Returns the row sums reduced over the half-wave (NR = 8: lane 4r holds row r0 + r; NR = 4: lane 8r) or,
// for dequantization, stores the rows; MODE kRowIndex records the row index (positions of rows 2, 4, 6) instead.
// Fully unrolled: every row's raw bytes live in their own registers.
// The row sums are formed one row behind the decode: row r's table entries wait while row r + 1 is decoded, so a
// wave decodes its first two rows before it needs its first raw row, and each later raw row has two rows' decode
// time to arrive (Qwen3-4B sweep 1726 -> 1695 us per token; two rows behind measured slower, 1743 us).
template <int ELEM, int MODE, bool XBF16, int NR, class Tab>
__device__ __forceinline__ float rowsN(const Tab &s, const uint32_t *lane, uint32_t P0, const BlockArgs &a, const Shape &f,
                                       const XRegs<XBF16> &x, uint4 *ring, const Coord0 &c, uint32_t r0, uint32_t L) {
    constexpr int RING = ring_depth<MODE>();
    Seq<ELEM> S;
    S.init_at(lane, P0);
    float acc[NR];
    if constexpr (MODE == kToken || MODE == kF32) {
        uint32_t e1[2][4], e2[2][4];                          // entries of rows r (slot r & 1) and r + 1
        row_codes(S, s, e1[0], e2[0]);
#pragma unroll
        for (int r = 0; r < NR; r++) {
            if (r + 1 < NR) row_codes(S, s, e1[(r + 1) & 1], e2[(r + 1) & 1]);
            const float sum = row_dot<MODE, XBF16>(e1[r & 1], e2[r & 1], ring[r % kRing0], x);
            if (r + kRing0 < NR) ring[r % kRing0] = raw_row<ELEM>(a.low, f, c, r + kRing0);
            acc[r] = c.col_ok ? sum : 0.f;
        }
        if constexpr (NR == 8) return reduce8_transposed(acc, L);
        else if constexpr (NR == 4) return reduce4_transposed(acc, L);
        else return reduce2_transposed(acc, L);
    }
#pragma unroll
    for (int r = 0; r < NR; r++) {
        if (MODE == kRowIndex && r > 0 && (r & 1) == 0)
            ((uint16_t *)a.out)[((uint64_t)c.b * kRowIndexSplits + (r >> 1) - 1) * kLanes + L] = (uint16_t)S.position(lane);
        uint32_t pw[8];
        const float sum = row0<ELEM, MODE, XBF16>(S, s, ring[r % RING], x, pw);
        // eight rows go through a ring of RING registers: row r + RING is requested when row r is done
        if (MODE != kRowIndex && r + RING < NR) ring[r % RING] = raw_row<ELEM>(a.low, f, c, r + RING);
        if (MODE == kDequant) store_row0<MODE>(a, f, c.row0 + r0 + r, c.col0, c.col_ok, pw);
        else acc[r] = c.col_ok ? sum : 0.f;
    }
    if (MODE == kDequant || MODE == kRowIndex) return 0.f;
    if constexpr (NR == 8) return reduce8_transposed(acc, L);
    else if constexpr (NR == 4) return reduce4_transposed(acc, L);
    else return reduce2_transposed(acc, L);
}

// rows0 for the pipelined kernel.  The raw-plane rows go through a ring of four registers (row r + 4 of this block
// is requested when row r is done, then rows 0-3 of the next block `nx`); at row 4 the next round's stream chunks and
// the next block's activations are requested.  `valid` is false for a half-wave without a block in the last round
// (it decodes a copy of the tile's last block and stores nothing).
template <int ELEM, int MODE, bool XBF16>
__device__ __forceinline__ float rows0_ring(const LutLds &s, const uint32_t *words, const BlockArgs &a, const Shape &f,
                                            const XRegs<XBF16> &x, uint4 ring[4], const Coord0 &c, const Coord0 &nx,
                                            bool valid, Bulk &Bk, const Region &Rn, XRegs<XBF16> &xn, uint32_t tid,
                                            uint32_t nth, uint32_t L) {
    Seq<ELEM> S;
    S.init(words);
    float acc[8];
#pragma unroll
    for (int r = 0; r < (int)kRows0; r++) {
        if (r == 4) {
            bulk_issue(Bk, a.data, Rn, tid, nth);
            if (MODE == kToken || MODE == kF32) load_x16<XBF16>(xn, a.x, nx.col0, nx.col_ok);
        }
        if (MODE == kRowIndex && r > 0 && (r & 1) == 0 && valid)
            ((uint16_t *)a.out)[((uint64_t)c.b * kRowIndexSplits + (r >> 1) - 1) * kLanes + L] = (uint16_t)S.position(words);
        uint32_t pw[8];
        const float sum = row0<ELEM, MODE, XBF16>(S, s, ring[r & 3], x, pw);
        if (MODE != kRowIndex)
            ring[r & 3] = r < 4 ? raw_row<ELEM>(a.low, f, c, r + 4) : raw_row<ELEM>(a.low, f, nx, r - 4);
        if (MODE == kDequant) store_row0<MODE>(a, f, valid ? c.row0 + r : f.M, c.col0, c.col_ok, pw);
        else acc[r] = c.col_ok ? sum : 0.f;
    }
    return MODE == kDequant || MODE == kRowIndex ? 0.f : reduce8_transposed(acc, L);
}

// The same for a block of a round whose streams do not fit the region buffer: decoded straight from global memory
// with a rolled row loop and its own raw loads (compact code; such rounds are rare, e.g. near-uniform exponent
// distributions).  Lanes past K16 have empty streams; the callers point them at the block's first word: decoding zero
// bits walks at most 96 words (all escapes), less than one block of such a round.
template <int ELEM, int MODE, bool XBF16, class Tab>
__device__ __forceinline__ float rows0_global(const Tab &s, const uint32_t *words, const BlockArgs &a, const Shape &f,
                                              const XRegs<XBF16> &x, const Coord0 &c, bool valid, uint32_t L) {
    Seq<ELEM> S;
    S.init(words);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int r = 0; r < (int)kRows0; r++) {
        if (MODE == kRowIndex && r > 0 && (r & 1) == 0 && valid)
            ((uint16_t *)a.out)[((uint64_t)c.b * kRowIndexSplits + (r >> 1) - 1) * kLanes + L] = (uint16_t)S.position(words);
        const uint4 cur = MODE == kRowIndex ? make_uint4(0u, 0u, 0u, 0u) : raw_row<ELEM>(a.low, f, c, r);
        uint32_t pw[8];
        const float sum = row0<ELEM, MODE, XBF16>(S, s, cur, x, pw);
        if (MODE == kDequant) {
            store_row0<MODE>(a, f, valid ? c.row0 + r : f.M, c.col0, c.col_ok, pw);
        } else {
#pragma unroll
            for (int i = 0; i < (int)kRows0 - 1; i++) acc[i] = acc[i + 1];    // rotation: at the end acc[i] = row i
            acc[kRows0 - 1] = c.col_ok ? sum : 0.f;
        }
    }
    return MODE == kDequant || MODE == kRowIndex ? 0.f : reduce8_transposed(acc, L);
}

// rowsN for a half-wave share of a block whose round does not fit the region buffer: from global memory, rolled.
template <int ELEM, int MODE, bool XBF16, int NR, class Tab>
__device__ __forceinline__ float rowsN_global(const Tab &s, const uint32_t *lane, uint32_t P0, const BlockArgs &a,
                                              const Shape &f, const XRegs<XBF16> &x, const Coord0 &c, uint32_t r0, uint32_t L) {
    Seq<ELEM> S;
    S.init_at(lane, P0);
    float acc[NR];
#pragma unroll
    for (int i = 0; i < NR; i++) acc[i] = 0.f;
#pragma unroll 1
    for (int r = 0; r < NR; r++) {
        const uint4 cur = raw_row<ELEM>(a.low, f, c, r);
        uint32_t pw[8];
        const float sum = row0<ELEM, MODE, XBF16>(S, s, cur, x, pw);
        if (MODE == kDequant) {
            store_row0<MODE>(a, f, c.row0 + r0 + r, c.col0, c.col_ok, pw);
        } else {
#pragma unroll
            for (int i = 0; i < NR - 1; i++) acc[i] = acc[i + 1];
            acc[NR - 1] = c.col_ok ? sum : 0.f;
        }
    }
    if (MODE == kDequant || MODE == kRowIndex) return 0.f;
    if constexpr (NR == 8) return reduce8_transposed(acc, L);
    else if constexpr (NR == 4) return reduce4_transposed(acc, L);
    else return reduce2_transposed(acc, L);
}

// Layout 0.  A workgroup owns G whole row groups (nt = G * CB blocks) and works through them in rounds of H blocks,
// one per half-wave; a round's streams are staged once into a region buffer of slot_words * H words.
//   PIPE = false (tiles of at most H blocks, small matrices; the launch plan guarantees it): every input is
//     requested before the decode table is staged, then one copy of the tile's streams.
//   PIPE = true: two region buffers; while round k decodes, round k + 1's streams, raw rows (four-register ring) and
//     activations are in flight and round k + 2's bounds and header bytes are read, so after the first round no step
//     waits on global memory.  One barrier per round publishes the next region.
// Staging of the decode table: the stored 12-bit LUT, re-encoded (PEEK 12), or the prepared 13-bit table (PEEK 13).
template <int PEEK> struct TabStage;
// issue: the first chunks of the decode table; commit: store them; finish: the chunks a small workgroup has left,
// called after every request that must not wait for the streams (lut_finish says why)
template <> struct TabStage<kPeek> {
    LutLoad Q;
    __device__ __forceinline__ void issue(const BlockArgs &a, uint32_t nth = blockDim.x) { lut_issue(Q, a.lut, nth); }
    __device__ __forceinline__ void commit(LutLds &s, uint32_t nth = blockDim.x) { lut_commit<kLutSeq>(s, Q, nth); }
    __device__ __forceinline__ void finish(LutLds &s, const BlockArgs &a, uint32_t nth = blockDim.x) {
        lut_finish<kLutSeq>(s, a.lut, nth);
    }
};
template <> struct TabStage<kPeekSeq> {
    SeqLoad Q;
    __device__ __forceinline__ void issue(const BlockArgs &a, uint32_t nth = blockDim.x) { seq_issue(Q, a.seq, nth); }
    __device__ __forceinline__ void commit(LutLds13 &s, uint32_t nth = blockDim.x) { seq_commit(s, Q, nth); }
    __device__ __forceinline__ void finish(LutLds13 &s, const BlockArgs &a, uint32_t nth = blockDim.x) {
        seq_finish(s, a.seq, nth);
    }
};

// nth: the workgroup's threads; flags: which of scale / bias are set (kFinishAll: read the pointers), for the token
// kernels whose arguments the hardware preloads (k_layout0p, k_layout0t) and which therefore read neither blockDim nor
// those pointers from memory before their first requests.  rg0: the tile's first row group.  PART: the workgroup
// decodes only rows NR jfix .. NR jfix + NR - 1 of its single row group (one half-wave per block, from the row
// index's position), for the split tail of k_layout0t.  s / dyn: the kernel's table and dynamic LDS.
template <int ELEM, int MODE, bool XBF16, bool PIPE, int NR, int PEEK, bool PART = false>
__device__ __forceinline__ void layout0_body(BlockArgs a, uint32_t nth, uint32_t flags, uint32_t rg0, uint32_t jfix,
                                             LutT<PEEK> &s, uint32_t *dyn) {
    static_assert(NR == 8 || ((NR == 4 || NR == 2) && !PIPE), "row splits only in the single-round kernel");
    static_assert(PEEK == kPeek || !PIPE, "the 13-bit table only in the single-round kernel");
    static_assert(!PART || (NR < 8 && !PIPE && (MODE == kToken || MODE == kDequant)),
                  "a row part of a single row group, token path or dequantization");
    constexpr uint32_t SP = PART ? 1u : kRows0 / NR;         // half-waves per block
    constexpr bool ROWS = MODE == kToken || MODE == kF32;     // modes that keep row sums
    const uint32_t tid = threadIdx.x, L = tid & 31;
    const uint32_t hw = tid >> 5, H = nth >> 5;
    const uint32_t HB = H / SP;                               // blocks per round
    const Shape f(a.M, a.K, 0);
    // words per region buffer: the tile's blocks (one round) or a round's (PIPE)
    const uint32_t cap = a.slot_words * (PIPE ? HB : min(HB, a.G * f.CB));
    uint32_t *cur = dyn, *nxt = dyn + cap;
    float *part = (float *)(dyn + (PIPE ? 2u : 1u) * cap);
    const uint32_t ng = min(a.G, f.groups() - rg0);
    const uint32_t nt = ng * f.CB, tl = nt - 1u;              // look-ahead past the tile re-reads block tl
    const uint32_t B0 = rg0 * f.CB, nb = f.nb;
    const uint32_t mend = !a.stride && B0 + nt == nb ? matrix_end(a, nb) : 0u;
    // request order: region bounds (none with fixed slots) and table first, then the stream copy (which needs the
    // bounds), then the activations and the raw rows; loads complete in order, so each wait below covers only what it
    // needs
    uint32_t t = hw / SP;
    const uint32_t r0 = PART ? NR * jfix : (hw % SP) * NR;    // first row of this half-wave's share of the block
    Coord0 c = coord0(min(t, tl), rg0, f, L);
    Region R = region_of(a, B0, B0 + min(HB, nt), nb, mend, a.stride);
    if constexpr (!PIPE) {
        // the block index and raw-plane offsets from this half-wave's first row on, computed before any vector load
        // is requested: the compiler may use a register with a load in flight as the don't-care high half of a 64-bit
        // multiply-add operand (c.b's), and would then wait for that load.  (After the scalar loads of the region
        // bounds: the empty asm counts as a memory write, which would turn later uniform loads into vector loads.)
        c.rb += r0 * f.K16;
        asm volatile("" : "+v"(c.rb), "+v"(c.b));
    }
    TabStage<PEEK> Q;
    Q.issue(a, nth);
    uint32_t n = a.hdr[(uint64_t)c.b * kHdrBytes + L], base = block_base(a, c.b);
    Bulk Bk;
    bulk_issue(Bk, a.data, R, tid, nth);
    XRegs<XBF16> x;
    if (ROWS) load_x16<XBF16>(x, a.x, c.col0, c.col_ok);
    // the finish's scale and bias after the streams: the preloaded kernels read those pointers from their argument
    // struct, and the wait for that read must not hold back the requests above
    const RowFinish fin = PART ? row_finish_load<MODE>(a, rg0 * kRows0 + r0, NR, flags)
                               : row_finish_load<MODE>(a, rg0 * kRows0, ng * kRows0, flags);

    if constexpr (!PIPE) {
        // everything but the raw rows is requested before the first wait; rows 0-1 once the workgroup's streams are
        // in, since the first raw row is needed only after two rows' decode (requested together with the streams
        // they delay them: o_proj 8.1 -> 8.7 us, qkv 9.1 -> 9.6; after this wave's own chunks, before the barrier:
        // 4B sweep 0.2% slower)
        const uint32_t P0 = NR == 8 ? 0u : part_start(a, c.b, r0 >> 1, L);
        Q.commit(s, nth);
        Q.finish(s, a, nth);
        const bool fits = R.n16 * 4u <= cap;
        if (fits) bulk_commit(Bk, cur, R, tid, nth);
        constexpr int RING = ring_depth<MODE>();
        uint4 raw[RING];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < (NR < RING ? NR : RING); r++)
            raw[r] = MODE == kRowIndex ? make_uint4(0u, 0u, 0u, 0u) : raw_row<ELEM>(a.low, f, c, r);
        if (t < nt) {
            const uint32_t start = c.col_ok ? half_scan_incl(n, L) - n : 0u;
            float v;
            if (fits) v = rowsN<ELEM, MODE, XBF16, NR>(s, cur + ((base - R.lo16) >> 2) + start, P0, a, f, x, raw, c, r0, L);
            else if constexpr (NR == 8)
                v = rows0_global<ELEM, MODE, XBF16>(s, (const uint32_t *)(a.data + base) + start, a, f, x, c, true, L);
            else
                v = rowsN_global<ELEM, MODE, XBF16, NR>(s, (const uint32_t *)(a.data + base) + start, P0, a, f, x, c, r0, L);
            // lane 4r (NR = 8), 8r (4) or 16r (2) holds row r0 + r
            if (ROWS && (L & (32u / NR - 1u)) == 0) part[(c.g * kRows0 + r0 + L / (32u / NR)) * f.CB + c.cb] = v;
        }
    } else {
        uint4 ring[4];
#pragma unroll
        for (int r = 0; r < 4; r++) ring[r] = MODE == kRowIndex ? make_uint4(0u, 0u, 0u, 0u) : raw_row<ELEM>(a.low, f, c, r);
        Coord0 cn = coord0(min(t + H, tl), rg0, f, L);
        uint32_t n_n = a.hdr[(uint64_t)cn.b * kHdrBytes + L], base_n = block_base(a, cn.b);
        Region Rn = region_of(a, B0 + min(H, tl), B0 + min(2u * H, nt), nb, mend, a.stride);
        Q.commit(s, nth);
        Q.finish(s, a, nth);
        if (R.n16 * 4u <= cap) bulk_commit(Bk, cur, R, tid, nth);
        __syncthreads();
        const uint32_t rounds = (nt + H - 1u) / H;
        uint32_t start = c.col_ok ? half_scan_incl(n, L) - n : 0u;
        for (uint32_t k = 0;; k++) {
            // round k + 2: this half-wave's header byte and base, and the region bounds
            const Coord0 cnn = coord0(min(t + 2u * H, tl), rg0, f, L);
            const uint32_t n_nn = a.hdr[(uint64_t)cnn.b * kHdrBytes + L], base_nn = block_base(a, cnn.b);
            const Region Rnn = region_of(a, B0 + min((k + 2u) * H, tl), B0 + min((k + 3u) * H, nt), nb, mend, a.stride);
            const bool valid = t < nt;
            XRegs<XBF16> xn;
            float v;
            if (R.n16 * 4u <= cap) {
                v = rows0_ring<ELEM, MODE, XBF16>(s, cur + ((base - R.lo16) >> 2) + start, a, f, x, ring, c, cn, valid, Bk,
                                                  Rn, xn, tid, nth, L);
            } else {
                bulk_issue(Bk, a.data, Rn, tid, nth);
                if (ROWS) load_x16<XBF16>(xn, a.x, cn.col0, cn.col_ok);
                v = rows0_global<ELEM, MODE, XBF16>(s, (const uint32_t *)(a.data + base) + start, a, f, x, c, valid, L);
#pragma unroll
                for (int r = 0; r < 4; r++) ring[r] = MODE == kRowIndex ? make_uint4(0u, 0u, 0u, 0u) : raw_row<ELEM>(a.low, f, cn, r);
            }
            if (valid && ROWS && (L & 3) == 0) part[(c.g * kRows0 + (L >> 2)) * f.CB + c.cb] = v;
            if (k + 1u >= rounds) break;
            if (Rn.n16 * 4u <= cap) bulk_commit(Bk, nxt, Rn, tid, nth);
            __syncthreads();                                     // region k + 1 visible; region k free
            uint32_t *tmp = cur; cur = nxt; nxt = tmp;
            start = cn.col_ok ? half_scan_incl(n_n, L) - n_n : 0u;
            base = base_n;
            R = Rn;
            Rn = Rnn;
            if (ROWS) x = xn;
            c = cn;
            cn = cnn;
            n_n = n_nn;
            base_n = base_nn;
            t += H;
        }
    }
    if (PART && ROWS) finish_rows<MODE>(a, part + r0 * f.CB, rg0 * kRows0 + r0, NR, f.CB, &fin, nth);
    else if (ROWS) finish_rows<MODE>(a, part, rg0 * kRows0, ng * kRows0, f.CB, &fin, nth);
}

template <int ELEM, int MODE, bool XBF16, bool PIPE, int NR, int PEEK = kPeek>
__global__ void __launch_bounds__(1024) k_layout0(BlockArgs a) {
    __shared__ LutT<PEEK> s;
    extern __shared__ uint32_t dyn[];
    layout0_body<ELEM, MODE, XBF16, PIPE, NR, PEEK>(a, blockDim.x, kFinishAll, blockIdx.x * a.G, 0u, s, dyn);
}

// The single-round kernel with the 13-bit table (token path with BF16 x, or dequantization: MODE) with the inputs of
// its first requests as leading scalar arguments, which gfx950 preloads into SGPRs (the library is built with
// -amdgpu-kernarg-preload-count): no wave waits for a kernarg read before requesting the table, header bytes,
// activations and streams (4B sweep 1685 -> 1644 us per token).  The eight arguments fill the 14 SGPRs gfx950 preloads next to the kernarg pointer; the row index, whose
// first use comes after the streams are in LDS, is read from `a`.  With fixed slots the stream copy needs only `data`
// and pk; otherwise it waits for the region bounds read from `bases`.
// pk = G | H << 16 | stride / 16 << 22 | has_scale << 30 | has_bias << 31, H = the workgroup's half-waves (at most
// 32), stride = the fixed-slot stride or 0; everything else comes from `a`, whose copies of these fields are ignored.
__device__ __forceinline__ void take_preloaded(BlockArgs &a, const uint8_t *data, const uint32_t *bases,
                                               const uint32_t *seq, uint32_t M, uint32_t K, uint32_t pk,
                                               const uint8_t *hdr, const void *xp) {
    a.data = data; a.bases = bases; a.seq = seq; a.M = M; a.K = K; a.hdr = hdr; a.x = xp;
    a.stride = ((pk >> 22) & 0xFFu) * 16u;
}
template <int ELEM, int NR, int MODE = kToken>
__global__ void __launch_bounds__(1024) k_layout0p(const uint8_t *__restrict__ data, const uint32_t *__restrict__ bases,
                                                   const uint32_t *__restrict__ seq, uint32_t M, uint32_t K, uint32_t pk,
                                                   const uint8_t *__restrict__ hdr, const void *__restrict__ xp,
                                                   BlockArgs a) {
    __shared__ LutT<kPeekSeq> s;
    extern __shared__ uint32_t dyn[];
    take_preloaded(a, data, bases, seq, M, K, pk, hdr, xp);
    a.G = pk & 0xFFFFu;
    layout0_body<ELEM, MODE, true, false, NR, kPeekSeq>(a, ((pk >> 16) & 0x3Fu) * 32u, pk >> 30, blockIdx.x * a.G, 0u,
                                                        s, dyn);
}

// Layout-0 token path and dequantization for matrices of one to two row groups per CU (k_layout0t): the first nfull
// workgroups (one per CU) take a whole row group each (NRF rows per half-wave, as k_layout0p); the TS-way parts (rows
// 8 / TS each, from the row index) of the remaining row groups go one to a workgroup, so every CU decodes about the
// same rows instead of some CUs two whole row groups (Qwen3-4B down and o_proj: 320 row groups on 256 CUs).  A part's
// workgroup stages its row group's streams whole, so those streams are read TS times (from L2 / the MALL after the
// first).  pk = nfull | H << 16 | stride / 16 << 22 | has_scale << 30 | has_bias << 31 (scale and bias: token path
// only; stride as for k_layout0p).
template <int ELEM, int NRF, int TS, int MODE = kToken>
__global__ void __launch_bounds__(1024) k_layout0t(const uint8_t *__restrict__ data, const uint32_t *__restrict__ bases,
                                                   const uint32_t *__restrict__ seq, uint32_t M, uint32_t K, uint32_t pk,
                                                   const uint8_t *__restrict__ hdr, const void *__restrict__ xp,
                                                   BlockArgs a) {
    static_assert(TS == 2 || TS == 4, "halves or quarters of a row group");
    static_assert(MODE == kToken || MODE == kDequant, "token path or dequantization");
    __shared__ LutT<kPeekSeq> s;
    extern __shared__ uint32_t dyn[];
    take_preloaded(a, data, bases, seq, M, K, pk, hdr, xp);
    a.G = 1;
    const uint32_t nfull = pk & 0xFFFFu, nth = ((pk >> 16) & 0x3Fu) * 32u, flags = pk >> 30;
    if (blockIdx.x < nfull) {
        layout0_body<ELEM, MODE, true, false, NRF, kPeekSeq>(a, nth, flags, blockIdx.x, 0u, s, dyn);
    } else {
        const uint32_t q = blockIdx.x - nfull;
        layout0_body<ELEM, MODE, true, false, 8 / TS, kPeekSeq, true>(a, nth, flags, nfull + q / TS, q % TS, s, dyn);
    }
}

template <int ELEM, int NRF, int TS, int MODE>
static void launch_layout0t(const LaunchPlan &p, const BlockArgs &a, hipStream_t st) {
    const uint32_t pk = p.G | ((p.threads / 32u) << 16) | ((a.stride >> 4) << 22) | (a.scale ? 1u << 30 : 0u) |
                        (a.bias ? 1u << 31 : 0u);
    hipLaunchKernelGGL((k_layout0t<ELEM, NRF, TS, MODE>), dim3(p.grid), dim3(p.threads), p.lds, st, a.data, a.bases,
                       a.seq, a.M, a.K, pk, a.hdr, a.x, a);
}

// the split-tail plan's kernel by rows per half-wave of a whole row group (8 / split) and parts per row group
template <int ELEM, int MODE>
static int launch_layout0_tail(const LaunchPlan &p, const BlockArgs &a, hipStream_t st) {
    const uint32_t nrf = 8u / p.split;
    if (p.tail == 4) {
        if (nrf == 2) launch_layout0t<ELEM, 2, 4, MODE>(p, a, st);
        else if (nrf == 4) launch_layout0t<ELEM, 4, 4, MODE>(p, a, st);
        else launch_layout0t<ELEM, 8, 4, MODE>(p, a, st);
    } else {
        if (nrf == 2) launch_layout0t<ELEM, 2, 2, MODE>(p, a, st);
        else if (nrf == 4) launch_layout0t<ELEM, 4, 2, MODE>(p, a, st);
        else launch_layout0t<ELEM, 8, 2, MODE>(p, a, st);
    }
    return (int)hipGetLastError();
}

template <int ELEM, int NR, int MODE = kToken>
static void launch_layout0p(const LaunchPlan &p, const BlockArgs &a, hipStream_t st) {
    const uint32_t pk = p.G | ((p.threads / 32u) << 16) | ((a.stride >> 4) << 22) | (a.scale ? 1u << 30 : 0u) |
                        (a.bias ? 1u << 31 : 0u);
    hipLaunchKernelGGL((k_layout0p<ELEM, NR, MODE>), dim3(p.grid), dim3(p.threads), p.lds, st, a.data, a.bases, a.seq,
                       a.M, a.K, pk, a.hdr, a.x, a);
}

// ---------------------------------------------------------------------------------------------------------------
// Layout 1: lane L = (r = L >> 2, q = L & 3) holds, per 32-column super-chunk, columns 8q..8q+7 of rows r and r+8.
// Stream positions 4k..4k+3 of a super-chunk are (row r, cols 2k, 2k+1) then (row r+8, cols 2k, 2k+1), so the four
// codes of one window step pair with raw word k and with activation pair k of the lane's 16-byte x slice.
template <int ELEM>
__device__ __forceinline__ uint4 raw_slot1(const uint8_t *__restrict__ p) {
    if (ELEM == kElemFp8) return expand_nibbles(ldnt2(p));
    return ldnt4(p);
}

// One layout-1 block for one lane: returns (row r sum, row r+8 sum) reduced over the lane's quad, or stores the rows.
template <int ELEM, int MODE, bool XBF16, typename P>
__device__ __forceinline__ float2 rows1(const LutLds &s, P words, const BlockArgs &a, const Shape &f, const uint8_t *rp,
                                        uint4 nxt, uint32_t nsc, uint32_t row0, uint32_t cb, uint32_t r, uint32_t q) {
    constexpr uint32_t RB = ELEM == kElemFp8 ? 8u : 16u;
    Window<ELEM, P> W;
    W.init(words);
    float accA = 0.f, accB = 0.f;
    for (uint32_t sc = 0; sc < nsc; sc++) {
        const uint4 cur = nxt;
        if (sc + 1 < nsc) nxt = raw_slot1<ELEM>(rp + (uint64_t)(sc + 1) * kLanes * RB);
        const uint32_t kc = cb * kCols + sc * 32 + 8 * q;
        uint4 xv = make_uint4(0, 0, 0, 0);
        float xf[8];
        if (MODE != kDequant) {
            if (XBF16) xv = *(const uint4 *)((const uint16_t *)a.x + kc);
            else {
                const float4 x0 = ((const float4 *)((const float *)a.x + kc))[0], x1 = ((const float4 *)((const float *)a.x + kc))[1];
                xf[0] = x0.x; xf[1] = x0.y; xf[2] = x0.z; xf[3] = x0.w; xf[4] = x1.x; xf[5] = x1.y; xf[6] = x1.z; xf[7] = x1.w;
            }
        }
        uint32_t pa[4], pb[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t e1, e2;
            W.quad(s, e1, e2);
            const uint32_t rk = u4_get(cur, k);
            if (MODE == kDequant) {
                pa[k] = perm(e1, rk, kSelPair0);
                pb[k] = perm(e2, rk, kSelPair2);
            } else if (XBF16) {
                const uint32_t xk = u4_get(xv, k);
                accA = dot2_bf16(perm(e1, rk, kSelPair0), xk, accA);
                accB = dot2_bf16(perm(e2, rk, kSelPair2), xk, accB);
            } else {
                accA = fmaf(__uint_as_float(perm(e1, rk, sel_f32(0, 5))), xf[2 * k], accA);
                accA = fmaf(__uint_as_float(perm(e1, rk, sel_f32(1, 6))), xf[2 * k + 1], accA);
                accB = fmaf(__uint_as_float(perm(e2, rk, sel_f32(2, 5))), xf[2 * k], accB);
                accB = fmaf(__uint_as_float(perm(e2, rk, sel_f32(3, 6))), xf[2 * k + 1], accB);
            }
        }
        if (MODE == kDequant && kc < f.K16) {                  // a half super-chunk beyond K16 is filler
            uint16_t *o = (uint16_t *)a.out + (uint64_t)row0 * f.K16 + kc;
            if (row0 + r < f.M) *(uint4 *)(o + (uint64_t)r * f.K16) = make_uint4(pa[0], pa[1], pa[2], pa[3]);
            if (row0 + r + 8 < f.M) *(uint4 *)(o + (uint64_t)(r + 8) * f.K16) = make_uint4(pb[0], pb[1], pb[2], pb[3]);
        }
    }
    accA += xor_f<1>(accA); accA += xor_f<2>(accA);            // the four lanes of a row pair
    accB += xor_f<1>(accB); accB += xor_f<2>(accB);
    return make_float2(accA, accB);
}

template <int ELEM, int MODE, bool XBF16>
__global__ void __launch_bounds__(1024) k_layout1(BlockArgs a) {
    __shared__ LutLds s;
    extern __shared__ uint32_t dyn[];
    stage_lut<kLutWindow>(s, a.lut);
    constexpr uint32_t RB = ELEM == kElemFp8 ? 8u : 16u;           // raw bytes per lane and super-chunk
    const uint32_t tid = threadIdx.x, L = tid & 31, r = L >> 2, q = L & 3;
    const uint32_t hw = tid >> 5, nhw = blockDim.x >> 5;
    uint32_t *slot = dyn + hw * a.slot_words;
    float *part = (float *)(dyn + nhw * a.slot_words);
    const Shape f(a.M, a.K, 1);
    const uint32_t rg0 = blockIdx.x * a.G;
    const uint32_t ng = min(a.G, f.groups() - rg0);
    const RowFinish fin = row_finish_load<MODE, ELEM == kElemFp8>(a, rg0 * kRows12, ng * kRows12);
    const uint32_t nt = ng * f.CB;

    for (uint32_t t = hw; t < nt; t += nhw) {
        const uint32_t g = t / f.CB, cb = t - g * f.CB, rb = rg0 + g, b = rb * f.CB + cb;
        const uint32_t row0 = rb * kRows12;
        const uint32_t nsc = ((cb == f.CB - 1 ? f.nl : 32u) + 1) / 2;
        const uint8_t *rp = a.low + ((uint64_t)(rb * f.spr + cb * 16) * kLanes + L) * RB;
        const LaneSpan sp = lane_span(a.hdr, b, L);
        const uint32_t base = a.bases[b];
        const uint4 first = raw_slot1<ELEM>(rp);
        uint32_t sh;
        float2 v;
        if (stage_block(slot, a.slot_words, a.data, base, sp.total, L, sh))
            v = rows1<ELEM, MODE, XBF16>(s, (const uint32_t *)slot + sh + sp.start, a, f, rp, first, nsc, row0, cb, r, q);
        else
            v = rows1<ELEM, MODE, XBF16>(s, (const uint32_t *)(a.data + base) + sp.start, a, f, rp, first, nsc, row0, cb, r, q);
        if (MODE != kDequant && q == 0) {
            part[(g * kRows12 + r) * f.CB + cb] = v.x;
            part[(g * kRows12 + r + 8) * f.CB + cb] = v.y;
        }
    }
    if (MODE != kDequant) finish_rows<MODE>(a, part, rg0 * kRows12, ng * kRows12, f.CB, ELEM == kElemFp8 ? &fin : nullptr);
}

// ---------------------------------------------------------------------------------------------------------------
// Layout 1, single round: a workgroup owns G whole 16-row groups (nt = G * CB <= H / SP blocks); their streams are
// staged once into LDS like layout 0's, and each half-wave decodes super-chunks sc0 .. sc0 + NS - 1 of one block
// (SP = 16 / NS half-waves per block; with SP > 1 the row index gives each lane's bit position at super-chunk
// 4, 8, 12).  Raw super-chunks go through a ring of two registers (chunk s + 2 is requested when chunk s is done).  Partial row sums are kept per (row, column block, part) and summed in a fixed
// order by the workgroup.
struct Coord1 {
    uint32_t g, cb, b, rb, nsc;
    uint32_t ro;                // byte offset in `low` of the lane's raw bytes of super-chunk 0 of the block
};
template <int ELEM>
__device__ __forceinline__ Coord1 coord1(uint32_t t, uint32_t rg0, const Shape &f, uint32_t L) {
    constexpr uint32_t RB = ELEM == kElemFp8 ? 8u : 16u;
    Coord1 c;
    c.g = t / f.CB;
    c.cb = t - c.g * f.CB;
    c.rb = rg0 + c.g;
    c.b = c.rb * f.CB + c.cb;
    c.nsc = c.cb == f.CB - 1u ? f.nsl : 16u;
    c.ro = ((c.rb * f.spr + c.cb * 16u) * kLanes + L) * RB;
    return c;
}
// Raw super-chunk sc of a block; past the block's last super-chunk it re-reads the last, so loads stay unconditional.
// 32-bit offsets (the plane is below 4 GB: M * K16 < 2^32) keep one address register per load.
template <int ELEM>
__device__ __forceinline__ uint4 raw1(const uint8_t *__restrict__ low, const Coord1 &c, uint32_t sc) {
    constexpr uint32_t RB = ELEM == kElemFp8 ? 8u : 16u;
    return raw_slot1<ELEM>(low + (c.ro + min(sc, c.nsc - 1u) * (kLanes * RB)));
}
// Eight activations from kc as BF16 pairs (fp32 x: rounded to BF16, as the reference's fp32 path does for layouts
// 1/2).  x holds K32 values, so every coded super-chunk is in bounds.
template <bool XBF16>
__device__ __forceinline__ uint4 x8_at(const void *x, uint32_t kc) {
    if constexpr (XBF16) return *(const uint4 *)((const uint16_t *)x + kc);
    const float4 a = ((const float4 *)((const float *)x + kc))[0], b = ((const float4 *)((const float *)x + kc))[1];
    return make_uint4(f32_to_bf16_rne(a.x) | f32_to_bf16_rne(a.y) << 16, f32_to_bf16_rne(a.z) | f32_to_bf16_rne(a.w) << 16,
                      f32_to_bf16_rne(b.x) | f32_to_bf16_rne(b.y) << 16, f32_to_bf16_rne(b.z) | f32_to_bf16_rne(b.w) << 16);
}
// The activations are staged once per workgroup as BF16 in LDS, so their per-super-chunk reads are LDS reads: a global
// load there would be waited for in issue order together with the raw chunks requested before it.
// In three parts, as the decode table is staged: the first two chunks per thread are requested with the prologue's
// other loads (x_issue) and stored after the table (x_commit; storing them waits for every load requested before
// them, the streams included); x_finish copies the rest (fewer than n8 / 2 threads).
template <bool XBF16> struct XStage { uint4 v0, v1; };
template <bool XBF16>
__device__ __forceinline__ void x_issue(XStage<XBF16> &X, const void *x, uint32_t n8, uint32_t tid, uint32_t nth) {
    X.v0 = x8_at<XBF16>(x, 8u * min(tid, n8 - 1u));
    X.v1 = x8_at<XBF16>(x, 8u * min(tid + nth, n8 - 1u));
}
template <bool XBF16>
__device__ __forceinline__ void x_commit(const XStage<XBF16> &X, uint4 *xs, uint32_t n8, uint32_t tid, uint32_t nth) {
    if (tid < n8) xs[tid] = X.v0;
    if (tid + nth < n8) xs[tid + nth] = X.v1;
}
template <bool XBF16>
__device__ __forceinline__ void x_finish(uint4 *xs, const void *x, uint32_t n8, uint32_t tid, uint32_t nth) {
    for (uint32_t i = tid + 2u * nth; i < n8; i += nth) xs[i] = x8_at<XBF16>(x, 8u * i);
}

// Raw super-chunks in flight per half-wave in the single-round kernel: two, as for layout 0's rows.
constexpr int kRing1 = 2;
// NEXT (NS = 4, several items per half-wave): each ring slot is refilled with the next item's super-chunk once used.
template <int ELEM, int MODE, int NS, bool FULL, bool NEXT = false, class Tab>
__device__ __forceinline__ float2 chunks1(const Tab &s, const uint32_t *lane, uint32_t P0, const BlockArgs &a,
                                          const Shape &f, const uint4 *xs, uint4 ring[4], const Coord1 &c, uint32_t sc0,
                                          uint32_t L, const Coord1 *cn = nullptr, uint32_t nsc0 = 0) {
    static_assert(!NEXT || NS == 4, "next-item refills for four-super-chunk items");
    constexpr int D = NEXT ? 4 : kRing1;                        // raw super-chunks in flight
    const uint32_t r = L >> 2, q = L & 3;
    Seq<ELEM> S;
    S.init_at(lane, P0);
    float accA = 0.f, accB = 0.f;
    const uint32_t kc0 = c.cb * kCols + 8u * q;
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const uint32_t sc = sc0 + i;
        if (!FULL && sc >= c.nsc) break;                        // the last column block codes nsl super-chunks
        if (MODE == kRowIndex && i > 0 && (i & 3) == 0)
            ((uint16_t *)a.out)[((uint64_t)c.b * kRowIndexSplits + (i >> 2) - 1) * kLanes + L] = (uint16_t)S.position(lane);
        uint4 xc = make_uint4(0u, 0u, 0u, 0u);
        if (MODE == kToken || MODE == kF32) xc = xs[(kc0 + sc * 32u) >> 3];
        const uint4 cw = ring[i % D];
        uint32_t pa[4], pb[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t s0 = S.s;
            const uint32_t *wp0 = S.wp;
            uint32_t e1, e2;
            if (__builtin_expect(__any(S.fast_quad(s, e1, e2) >= kSeqSlowTest), 0)) {
                S.s = s0;
                S.wp = wp0;
                S.reload();
                S.slow_quad(s, e1, e2);
            }
            const uint32_t rk = u4_get(cw, k);
            if (MODE == kDequant) {
                pa[k] = perm(e1, rk, kSelPair0);
                pb[k] = perm(e2, rk, kSelPair2);
                asm volatile("" : "+v"(pa[k]), "+v"(pb[k]));
            } else if (MODE == kToken || MODE == kF32) {
                const uint32_t xk = u4_get(xc, k);
                accA = dot2_bf16(perm(e1, rk, kSelPair0), xk, accA);
                accB = dot2_bf16(perm(e2, rk, kSelPair2), xk, accB);
                asm volatile("" : "+v"(accA), "+v"(accB));
            }
        }
        if constexpr (NEXT) ring[i % D] = raw1<ELEM>(a.low, *cn, nsc0 + i);
        else if (MODE != kRowIndex && i + D < NS) ring[i % D] = raw1<ELEM>(a.low, c, sc + (uint32_t)D);
        if (MODE == kDequant) {
            const uint32_t kc = kc0 + sc * 32u, row0 = c.rb * kRows12;
            if (kc < f.K16) {                                   // a half super-chunk beyond K16 is filler
                uint16_t *o = (uint16_t *)a.out + (uint64_t)row0 * f.K16 + kc;
                if (row0 + r < f.M) *(uint4 *)(o + (uint64_t)r * f.K16) = make_uint4(pa[0], pa[1], pa[2], pa[3]);
                if (row0 + r + 8 < f.M) *(uint4 *)(o + (uint64_t)(r + 8) * f.K16) = make_uint4(pb[0], pb[1], pb[2], pb[3]);
            }
        }
    }
    if (MODE == kRowIndex) {                                    // entries past the block's last super-chunk: its end
        for (uint32_t j = (c.nsc + 3u) / 4u; j <= kRowIndexSplits; j++)
            if (j >= 1u && 4u * j >= c.nsc)
                ((uint16_t *)a.out)[((uint64_t)c.b * kRowIndexSplits + j - 1u) * kLanes + L] = (uint16_t)S.position(lane);
    }
    accA += xor_f<1>(accA); accA += xor_f<2>(accA);              // the four lanes of a row pair
    accB += xor_f<1>(accB); accB += xor_f<2>(accB);
    return make_float2(accA, accB);
}

// chunks1 for a block whose tile does not fit the region buffer (and for building the row index): from global memory,
// with a rolled loop and one raw load per super-chunk (compact code for a rare path).
template <int ELEM, int MODE, int NS, class Tab>
__device__ __forceinline__ float2 chunks1_global(const Tab &s, const uint32_t *lane, uint32_t P0, const BlockArgs &a,
                                                 const uint4 *xs, const Coord1 &c, uint32_t sc0, uint32_t L) {
    Seq<ELEM> S;
    S.init_at(lane, P0);
    float accA = 0.f, accB = 0.f;
    const uint32_t kc0 = c.cb * kCols + 8u * (L & 3);
    const uint32_t sc1 = min(sc0 + NS, c.nsc);
#pragma unroll 1
    for (uint32_t sc = sc0; sc < sc1; sc++) {
        if (MODE == kRowIndex && sc > 0 && (sc & 3) == 0)
            ((uint16_t *)a.out)[((uint64_t)c.b * kRowIndexSplits + (sc >> 2) - 1) * kLanes + L] = (uint16_t)S.position(lane);
        const uint4 cw = MODE == kRowIndex ? make_uint4(0u, 0u, 0u, 0u) : raw1<ELEM>(a.low, c, sc);
        const uint4 xc = MODE == kToken || MODE == kF32 ? xs[(kc0 + sc * 32u) >> 3] : make_uint4(0u, 0u, 0u, 0u);
        uint32_t pa[4], pb[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t s0 = S.s;
            const uint32_t *wp0 = S.wp;
            uint32_t e1, e2;
            if (__builtin_expect(__any(S.fast_quad(s, e1, e2) >= kSeqSlowTest), 0)) {
                S.s = s0;
                S.wp = wp0;
                S.reload();
                S.slow_quad(s, e1, e2);
            }
            const uint32_t rk = u4_get(cw, k);
            if (MODE == kToken || MODE == kF32) {
                const uint32_t xk = u4_get(xc, k);
                accA = dot2_bf16(perm(e1, rk, kSelPair0), xk, accA);
                accB = dot2_bf16(perm(e2, rk, kSelPair2), xk, accB);
            } else if (MODE == kDequant) {
                pa[k] = perm(e1, rk, kSelPair0);
                pb[k] = perm(e2, rk, kSelPair2);
            }
        }
        if (MODE == kDequant) {                                 // as in chunks1
            const Shape f(a.M, a.K, 1);
            const uint32_t kc = kc0 + sc * 32u, row0 = c.rb * kRows12, r = L >> 2;
            if (kc < f.K16) {
                uint16_t *o = (uint16_t *)a.out + (uint64_t)row0 * f.K16 + kc;
                if (row0 + r < f.M) *(uint4 *)(o + (uint64_t)r * f.K16) = make_uint4(pa[0], pa[1], pa[2], pa[3]);
                if (row0 + r + 8 < f.M) *(uint4 *)(o + (uint64_t)(r + 8) * f.K16) = make_uint4(pb[0], pb[1], pb[2], pb[3]);
            }
        }
    }
    if (MODE == kRowIndex) {                                    // entries past the block's last super-chunk: its end
        for (uint32_t j = 1; j <= kRowIndexSplits; j++)
            if (4u * j >= c.nsc)
                ((uint16_t *)a.out)[((uint64_t)c.b * kRowIndexSplits + j - 1u) * kLanes + L] = (uint16_t)S.position(lane);
    }
    accA += xor_f<1>(accA); accA += xor_f<2>(accA);
    accB += xor_f<1>(accB); accB += xor_f<2>(accB);
    return make_float2(accA, accB);
}

template <int ELEM, int MODE, bool XBF16, int NS, bool FULL, int PEEK>
__device__ __forceinline__ void layout1s_body(BlockArgs a, uint32_t nth, uint32_t flags) {
    constexpr uint32_t SP = 16u / NS;                          // half-waves per block
    constexpr bool ROWS = MODE == kToken || MODE == kF32;
    __shared__ LutT<PEEK> s;
    extern __shared__ uint32_t dyn[];
    const uint32_t tid = threadIdx.x, L = tid & 31;
    const uint32_t hw = tid >> 5;
    const Shape f(a.M, a.K, 1);
    // Dequantization may take a range of blocks instead of whole row groups (bit 31 of G set, G & 0x7FFFFFFF blocks
    // per workgroup): with no row sums to combine, a tile may start and end inside a row group.
    const bool bt = MODE == kDequant && (a.G >> 31) != 0u;
    const uint32_t gsz = a.G & 0x7FFFFFFFu;
    const uint32_t cap = a.slot_words * (bt ? gsz : gsz * f.CB);   // the plan's region: one slot per block of the tile
    const uint32_t n8 = (f.K16 + 31u) / 32u * 4u;               // x: K32 BF16 values, in chunks of eight
    uint32_t *cur = dyn;
    uint4 *xs = (uint4 *)(dyn + cap);
    float *part = (float *)(xs + (ROWS ? n8 : 0u));
    const uint32_t nb = f.nb;
    const uint32_t rg0 = bt ? 0u : blockIdx.x * gsz;
    const uint32_t ng = bt ? 0u : min(gsz, f.groups() - rg0);
    const uint32_t B0 = bt ? blockIdx.x * gsz : rg0 * f.CB;
    const uint32_t nt = bt ? min(gsz, nb - B0) : ng * f.CB, tl = nt - 1u;
    const uint32_t mend = !a.stride && B0 + nt == nb ? matrix_end(a, nb) : 0u;
    Region R = region_of(a, B0, B0 + nt, nb, mend, a.stride);
    TabStage<PEEK> Q;
    Q.issue(a, nth);
    const uint32_t t = hw / SP, p = hw % SP, sc0 = p * NS;
    const Coord1 c = coord1<ELEM>((bt ? B0 : 0u) + min(t, tl), rg0, f, L);   // with bt: rg0 = 0, absolute block
    const uint32_t n = a.hdr[(uint64_t)c.b * kHdrBytes + L], base = block_base(a, c.b);
    Bulk Bk;
    bulk_issue(Bk, a.data, R, tid, nth);
    XStage<XBF16> X;
    if (ROWS) x_issue<XBF16>(X, a.x, n8, tid, nth);
    // fp8: the finish's row scale after the streams (the preloaded kernel reads its pointer from the argument struct,
    // and the wait for that read must not hold back the requests above)
    const RowFinish fin = row_finish_load<MODE, ELEM == kElemFp8>(a, rg0 * kRows12, ng * kRows12, flags);
    // the raw chunks are requested once this wave's stream chunks are in, before the barrier (the first one is used
    // by the first decode step)
    const uint32_t P0 = SP == 1 ? 0u : part_start(a, c.b, sc0 / 4u, L);
    Q.commit(s, nth);
    if (ROWS) {
        x_commit<XBF16>(X, xs, n8, tid, nth);
        x_finish<XBF16>(xs, a.x, n8, tid, nth);
    }
    Q.finish(s, a, nth);
    // the copy moves four 16-byte chunks per thread (512 words per half-wave); a larger region (one half-wave per
    // block, as when the row index is built) decodes from global memory, except for dequantization, which copies the
    // rest of its region in a second pass
    const bool fits = (MODE == kDequant || R.n16 <= 4u * nth) && R.n16 * 4u <= cap;
    if (fits) {
        bulk_commit(Bk, cur, R, tid, nth);
        if (MODE == kDequant)
            for (uint32_t i = tid + 4u * nth; i < R.n16; i += nth)
                *(u32x4_t *)(cur + 4u * i) = *(const u32x4_t *)(a.data + R.lo16 + 16u * i);
    }
    uint4 ring[4];
#pragma unroll
    for (int i = 0; i < kRing1; i++) ring[i] = MODE == kRowIndex ? make_uint4(0u, 0u, 0u, 0u) : raw1<ELEM>(a.low, c, sc0 + i);
    __syncthreads();
    if (t < nt) {
        const uint32_t start = half_scan_incl(n, L) - n;
        const uint32_t pi = ((c.g * kRows12 + (L >> 2)) * f.CB + c.cb) * SP + p;   // partial sum slot of row r
        float2 v = make_float2(0.f, 0.f);
        if (FULL || sc0 < c.nsc) {
            if (fits) v = chunks1<ELEM, MODE, NS, FULL>(s, cur + ((base - R.lo16) >> 2) + start, P0, a, f, xs, ring, c, sc0, L);
            else v = chunks1_global<ELEM, MODE, NS>(s, (const uint32_t *)(a.data + base) + start, P0, a, xs, c, sc0, L);
        }
        if (ROWS && (L & 3) == 0) {
            part[pi] = v.x;
            part[pi + 8u * f.CB * SP] = v.y;                   // row r + 8
        }
    }
    if (ROWS) finish_rows<MODE>(a, part, rg0 * kRows12, ng * kRows12, f.CB * SP, ELEM == kElemFp8 ? &fin : nullptr, nth);
}

template <int ELEM, int MODE, bool XBF16, int NS, bool FULL, int PEEK = kPeek>
__global__ void __launch_bounds__(1024) k_layout1s(BlockArgs a) {
    layout1s_body<ELEM, MODE, XBF16, NS, FULL, PEEK>(a, blockDim.x, kFinishAll);
}

// k_layout1s's token path with the inputs of its first requests preloaded into SGPRs (as k_layout0p; the table
// argument is the stored LUT for PEEK = 12).
template <int ELEM, int NS, bool FULL, int PEEK>
__global__ void __launch_bounds__(1024) k_layout1sp(const uint8_t *__restrict__ data, const uint32_t *__restrict__ bases,
                                                    const uint32_t *__restrict__ seq, uint32_t M, uint32_t K, uint32_t pk,
                                                    const uint8_t *__restrict__ hdr, const void *__restrict__ xp,
                                                    BlockArgs a) {
    take_preloaded(a, data, bases, seq, M, K, pk, hdr, xp);
    if (PEEK != kPeekSeq) a.lut = seq;                         // the table this kernel stages
    a.G = pk & 0xFFFFu;
    layout1s_body<ELEM, kToken, true, NS, FULL, PEEK>(a, ((pk >> 16) & 0x3Fu) * 32u, pk >> 30);
}

// Layout 1, several items per half-wave: for matrices whose row groups hold more blocks than a workgroup has
// half-waves at two per block (K > 8192, e.g. 2560 x 9728: 19 blocks per 16-row group).  A workgroup owns one 16-row
// group (its streams staged once, up to ~90 KB of LDS), and its items (block, quarter of the super-chunks) go
// round-robin to 32 half-waves; while an item decodes, the next item's raw super-chunks, header byte, base and
// row-index entry are requested, so a half-wave never waits for global memory between items.
template <int ELEM, bool FULL, int PEEK>
__device__ __forceinline__ void layout1m_body(BlockArgs a, uint32_t nth, uint32_t flags) {
    constexpr int MODE = kToken;
    constexpr uint32_t NS = 4, SP = 4;
    __shared__ LutT<PEEK> s;
    extern __shared__ uint32_t dyn[];
    const uint32_t tid = threadIdx.x, L = tid & 31;
    const uint32_t hw = tid >> 5, H = nth >> 5;
    const Shape f(a.M, a.K, 1);
    const uint32_t rg0 = blockIdx.x * a.G;
    const uint32_t ng = min(a.G, f.groups() - rg0);
    const uint32_t nt = ng * f.CB;
    const uint32_t cap = a.slot_words * a.G * f.CB;
    const uint32_t n8 = (f.K16 + 31u) / 32u * 4u;
    uint32_t *cur = dyn;
    uint4 *xs = (uint4 *)(dyn + cap);
    float *part = (float *)(xs + n8);
    const uint32_t B0 = rg0 * f.CB, nb = f.nb;
    const uint32_t mend = !a.stride && B0 + nt == nb ? matrix_end(a, nb) : 0u;
    Region R = region_of(a, B0, B0 + nt, nb, mend, a.stride);
    TabStage<PEEK> Q;
    Q.issue(a, nth);
    const uint32_t ntot = nt * SP, itl = ntot - 1u;
    auto item = [&](uint32_t it, Coord1 &c, uint32_t &p) {
        const uint32_t i = min(it, itl);
        c = coord1<ELEM>(i / SP, rg0, f, L);
        p = i % SP;
    };
    Coord1 c;
    uint32_t p;
    item(hw, c, p);
    uint32_t n = a.hdr[c.b * kHdrBytes + L], base = block_base(a, c.b);
    Bulk Bk;
    bulk_issue(Bk, a.data, R, tid, nth);
    // the row-index entry and (fp8) the finish's row scale after the streams: the preloaded kernel reads both
    // pointers from its argument struct, and the wait for that read must not hold back the stream copy
    uint32_t P0 = p ? a.aux[(c.b * kRowIndexSplits + p - 1u) * kLanes + L] : 0u;
    const RowFinish fin = row_finish_load<MODE, ELEM == kElemFp8>(a, rg0 * kRows12, ng * kRows12, flags);
    // the activations are stored first, which waits for the streams; then the table and the raw chunks (an order
    // measured faster here than k_layout1s's: 2560x9728 15.8 us against 16.6-17.0, the later ones leaving the
    // compiler a register choice that waits inside the item loop)
    XStage<true> X;
    x_issue<true>(X, a.x, n8, tid, nth);
    x_commit<true>(X, xs, n8, tid, nth);
    x_finish<true>(xs, a.x, n8, tid, nth);
    Q.commit(s, nth);
    Q.finish(s, a, nth);
    uint4 ring[4];
#pragma unroll
    for (int i = 0; i < 4; i++) ring[i] = raw1<ELEM>(a.low, c, p * NS + i);
    const bool fits = R.n16 <= 4u * nth && R.n16 * 4u <= cap;
    if (fits) bulk_commit(Bk, cur, R, tid, nth);
    __syncthreads();
    // trip count of the wave (both halves run it; a half without an item decodes a copy of the last and stores nothing)
    const uint32_t hw0 = hw & ~1u;
    const uint32_t nk = ntot > hw0 ? (ntot - hw0 + H - 1u) / H : 0u;
    uint32_t it = hw;
    for (uint32_t k = 0; k < nk; k++) {
        Coord1 cn;
        uint32_t pn;
        item(it + H, cn, pn);
        const uint32_t nn = a.hdr[cn.b * kHdrBytes + L], basen = block_base(a, cn.b);
        const uint32_t P0n = pn ? a.aux[(cn.b * kRowIndexSplits + pn - 1u) * kLanes + L] : 0u;
        const uint32_t start = half_scan_incl(n, L) - n, sc0 = p * NS;
        float2 v = make_float2(0.f, 0.f);
        if (FULL || sc0 < c.nsc) {
            if (fits)
                v = chunks1<ELEM, MODE, NS, FULL, true>(s, cur + ((base - R.lo16) >> 2) + start, P0, a, f, xs, ring, c, sc0, L,
                                                        &cn, pn * NS);
            else
                v = chunks1_global<ELEM, MODE, NS>(s, (const uint32_t *)(a.data + base) + start, P0, a, xs, c, sc0, L);
        }
        if (!fits || !(FULL || sc0 < c.nsc)) {
#pragma unroll
            for (int i = 0; i < 4; i++) ring[i] = raw1<ELEM>(a.low, cn, pn * NS + i);
        }
        if (it < ntot && (L & 3) == 0) {
            const uint32_t pi = ((c.g * kRows12 + (L >> 2)) * f.CB + c.cb) * SP + p;
            part[pi] = v.x;
            part[pi + 8u * f.CB * SP] = v.y;
        }
        it += H;
        c = cn;
        p = pn;
        n = nn;
        base = basen;
        P0 = P0n;
    }
    finish_rows<MODE>(a, part, rg0 * kRows12, ng * kRows12, f.CB * SP, ELEM == kElemFp8 ? &fin : nullptr, nth);
}

// The kernel, with the inputs of its first requests preloaded into SGPRs (as k_layout0p).
template <int ELEM, bool FULL, int PEEK>
__global__ void __launch_bounds__(1024) k_layout1mp(const uint8_t *__restrict__ data, const uint32_t *__restrict__ bases,
                                                    const uint32_t *__restrict__ seq, uint32_t M, uint32_t K, uint32_t pk,
                                                    const uint8_t *__restrict__ hdr, const void *__restrict__ xp,
                                                    BlockArgs a) {
    take_preloaded(a, data, bases, seq, M, K, pk, hdr, xp);
    if (PEEK != kPeekSeq) a.lut = seq;                         // the table this kernel stages
    a.G = pk & 0xFFFFu;
    layout1m_body<ELEM, FULL, PEEK>(a, ((pk >> 16) & 0x3Fu) * 32u, pk >> 30);
}

// ---------------------------------------------------------------------------------------------------------------
// Row gather: one half-wave per requested row.  Layout 0 decodes and discards the rows in front of it inside each
// column block; layout 1 decodes the whole 16-row group and the row's lanes store.
template <int ELEM, typename P>
__device__ __forceinline__ void gather_block0(const LutLds &s, P words, uint4 raw, uint32_t rr, uint16_t *o, uint32_t col0, bool col_ok) {
    Window<ELEM, P> W;
    W.init(words);
    for (uint32_t z = 0; z < rr; z++) {
#pragma unroll
        for (int k = 0; k < 4; k++) W.skip_quad(s);
    }
    uint32_t pw[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t e1, e2;
        W.quad(s, e1, e2);
        const uint32_t rk = u4_get(raw, k);
        pw[2 * k] = perm(e1, rk, kSelPair0);
        pw[2 * k + 1] = perm(e2, rk, kSelPair2);
    }
    if (col_ok) {
        uint4 *op = (uint4 *)(o + col0);
        op[0] = make_uint4(pw[0], pw[1], pw[2], pw[3]);
        op[1] = make_uint4(pw[4], pw[5], pw[6], pw[7]);
    }
}

template <int ELEM>
__global__ void __launch_bounds__(256) k_gather0(GatherArgs a) {
    __shared__ LutLds s;
    extern __shared__ uint32_t dyn[];
    stage_lut<kLutWindow>(s, a.lut);
    const uint32_t L = threadIdx.x & 31, hw = threadIdx.x >> 5;
    uint32_t *slot = dyn + hw * a.slot_words;
    const Shape f(a.M, a.K, 0);
    // one half-wave per (id, column block): the blocks of a row decode in parallel
    const uint32_t item = blockIdx.x * (blockDim.x >> 5) + hw, id = item / f.CB, cb = item - id * f.CB;
    if (id >= a.n_ids) return;
    const int64_t R = a.ids[id];
    if (R < 0 || R >= (int64_t)a.M) return;
    const uint32_t rb = (uint32_t)R / kRows0, rr = (uint32_t)R % kRows0;
    uint16_t *o = a.out + (uint64_t)id * f.K16;
    {
        const uint32_t b = rb * f.CB + cb, col0 = cb * kCols + L * 16;
        const bool col_ok = col0 < f.K16;
        const LaneSpan sp = lane_span(a.hdr, b, L);
        const uint32_t base = a.bases[b];
        const uint4 raw = raw_row0<ELEM>(a.low, f, (uint32_t)R, col0, col_ok);
        uint32_t sh;
        if (stage_block(slot, a.slot_words, a.data, base, sp.total, L, sh))
            gather_block0<ELEM>(s, (const uint32_t *)slot + sh + sp.start, raw, rr, o, col0, col_ok);
        else
            gather_block0<ELEM>(s, (const uint32_t *)(a.data + base) + sp.start, raw, rr, o, col0, col_ok);
    }
}

template <int ELEM, typename P>
__device__ __forceinline__ void gather_block1(const LutLds &s, P words, const uint8_t *rp, uint32_t nsc, bool mine, bool upper,
                                              uint16_t *o, uint32_t cb, uint32_t q, uint32_t K16) {
    constexpr uint32_t RB = ELEM == kElemFp8 ? 8u : 16u;
    Window<ELEM, P> W;
    W.init(words);
    for (uint32_t sc = 0; sc < nsc; sc++) {
        const uint4 raw = raw_slot1<ELEM>(rp + (uint64_t)sc * kLanes * RB);
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t e1, e2;
            W.quad(s, e1, e2);
            const uint32_t rk = u4_get(raw, k);
            v[k] = upper ? perm(e2, rk, kSelPair2) : perm(e1, rk, kSelPair0);
        }
        const uint32_t kc = cb * kCols + sc * 32 + 8 * q;
        if (mine && kc < K16) *(uint4 *)(o + kc) = make_uint4(v[0], v[1], v[2], v[3]);
    }
}

template <int ELEM>
__global__ void __launch_bounds__(256) k_gather1(GatherArgs a) {
    __shared__ LutLds s;
    extern __shared__ uint32_t dyn[];
    stage_lut<kLutWindow>(s, a.lut);
    constexpr uint32_t RB = ELEM == kElemFp8 ? 8u : 16u;
    const uint32_t L = threadIdx.x & 31, r = L >> 2, q = L & 3, hw = threadIdx.x >> 5;
    uint32_t *slot = dyn + hw * a.slot_words;
    const Shape f(a.M, a.K, 1);
    // one half-wave per (id, column block): the blocks of a row decode in parallel
    const uint32_t item = blockIdx.x * (blockDim.x >> 5) + hw, id = item / f.CB, cb = item - id * f.CB;
    if (id >= a.n_ids) return;
    const int64_t R = a.ids[id];
    if (R < 0 || R >= (int64_t)a.M) return;
    const uint32_t rb = (uint32_t)R / kRows12, rr = (uint32_t)R % kRows12;
    const bool mine = (rr & 7u) == r, upper = rr >= 8;
    uint16_t *o = a.out + (uint64_t)id * f.K16;
    {
        const uint32_t b = rb * f.CB + cb;
        const uint32_t nsc = ((cb == f.CB - 1 ? f.nl : 32u) + 1) / 2;
        const uint8_t *rp = a.low + ((uint64_t)(rb * f.spr + cb * 16) * kLanes + L) * RB;
        const LaneSpan sp = lane_span(a.hdr, b, L);
        const uint32_t base = a.bases[b];
        uint32_t sh;
        if (stage_block(slot, a.slot_words, a.data, base, sp.total, L, sh))
            gather_block1<ELEM>(s, (const uint32_t *)slot + sh + sp.start, rp, nsc, mine, upper, o, cb, q, f.K16);
        else
            gather_block1<ELEM>(s, (const uint32_t *)(a.data + base) + sp.start, rp, nsc, mine, upper, o, cb, q, f.K16);
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Layout 1 token path (BF16 x, row index): the multi-item kernel or the single-round kernel with a 4 or 8
// super-chunk split, with the stored 12-bit LUT or the 13-bit table.  FULL when every block codes all 16
// super-chunks (K a multiple of 512).
template <int ELEM, int PEEK>
static int launch_layout1_token(const LaunchPlan &p, const BlockArgs &a, hipStream_t st, bool full) {
    const dim3 g(p.grid), b(p.threads);
    // the preloaded kernels' packed word: tile, half-waves, slot stride, scale and bias present
    const uint32_t pk = p.G | ((p.threads / 32u) << 16) | ((a.stride >> 4) << 22) | (a.scale ? 1u << 30 : 0u) |
                        (a.bias ? 1u << 31 : 0u);
    // the table argument: the 13-bit table or the stored LUT, whichever the kernel stages
#define NWC_L1_PRELOAD a.data, a.bases, PEEK == kPeekSeq ? a.seq : a.lut, a.M, a.K, pk, a.hdr, a.x, a
    if (p.multi) {
        // more than 64 KB of LDS: raise the kernel's limit (idempotent, so concurrent first calls are fine)
        auto kf = full ? (const void *)k_layout1mp<ELEM, true, PEEK> : (const void *)k_layout1mp<ELEM, false, PEEK>;
        if (p.lds > 64u * 1024u) {
            const hipError_t e = hipFuncSetAttribute(kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)p.lds);
            if (e != hipSuccess) return (int)e;
        }
        if (full) hipLaunchKernelGGL((k_layout1mp<ELEM, true, PEEK>), g, b, p.lds, st, NWC_L1_PRELOAD);
        else hipLaunchKernelGGL((k_layout1mp<ELEM, false, PEEK>), g, b, p.lds, st, NWC_L1_PRELOAD);
        return (int)hipGetLastError();
    }
    if (p.split == 4 && p.G < 65536u) {
        if (full) hipLaunchKernelGGL((k_layout1sp<ELEM, 4, true, PEEK>), g, b, p.lds, st, NWC_L1_PRELOAD);
        else hipLaunchKernelGGL((k_layout1sp<ELEM, 4, false, PEEK>), g, b, p.lds, st, NWC_L1_PRELOAD);
        return (int)hipGetLastError();
    }
    if (p.split == 2 && p.G < 65536u) {
        if (full) hipLaunchKernelGGL((k_layout1sp<ELEM, 8, true, PEEK>), g, b, p.lds, st, NWC_L1_PRELOAD);
        else hipLaunchKernelGGL((k_layout1sp<ELEM, 8, false, PEEK>), g, b, p.lds, st, NWC_L1_PRELOAD);
        return (int)hipGetLastError();
    }
#undef NWC_L1_PRELOAD
    return -1;
}

// Layout 1, single round.
template <int ELEM, int MODE, bool XBF16, int NS, int PEEK>
static void launch_ns(bool full, dim3 g, dim3 b, uint32_t lds, hipStream_t st, const BlockArgs &a) {
    if (full) hipLaunchKernelGGL((k_layout1s<ELEM, MODE, XBF16, NS, true, PEEK>), g, b, lds, st, a);
    else hipLaunchKernelGGL((k_layout1s<ELEM, MODE, XBF16, NS, false, PEEK>), g, b, lds, st, a);
}

template <int ELEM, int MODE, bool XBF16>
static int launch_layout1s(const LaunchPlan &p, const BlockArgs &a, hipStream_t st) {
    const bool full = Shape(a.M, a.K, 1).nsl == 16u;
    const dim3 g(p.grid), b(p.threads);
    if constexpr (MODE == kToken && XBF16) {                   // the entry point that takes the row index and table
        if (p.seq13) return launch_layout1_token<ELEM, kPeekSeq>(p, a, st, full);
        return launch_layout1_token<ELEM, kPeek>(p, a, st, full);
    }
    if constexpr (MODE == kRowIndex) {
        if (p.split != 1) return -1;
        if (full) hipLaunchKernelGGL((k_layout1s<ELEM, MODE, XBF16, 16, true>), g, b, p.lds, st, a);
        else hipLaunchKernelGGL((k_layout1s<ELEM, MODE, XBF16, 16, false>), g, b, p.lds, st, a);
        return (int)hipGetLastError();
    }
    if constexpr (MODE == kDequant) {                          // one, two or four half-waves per block
        if (p.seq13) {
            if (p.split == 4) launch_ns<ELEM, MODE, XBF16, 4, kPeekSeq>(full, g, b, p.lds, st, a);
            else if (p.split == 2) launch_ns<ELEM, MODE, XBF16, 8, kPeekSeq>(full, g, b, p.lds, st, a);
            else launch_ns<ELEM, MODE, XBF16, 16, kPeekSeq>(full, g, b, p.lds, st, a);
        } else {
            if (p.split == 4) launch_ns<ELEM, MODE, XBF16, 4, kPeek>(full, g, b, p.lds, st, a);
            else if (p.split == 2) launch_ns<ELEM, MODE, XBF16, 8, kPeek>(full, g, b, p.lds, st, a);
            else launch_ns<ELEM, MODE, XBF16, 16, kPeek>(full, g, b, p.lds, st, a);
        }
        return (int)hipGetLastError();
    }
    return -1;
}

template <int ELEM, int MODE, bool XBF16>
static int launch_prefix_t(const LaunchPlan &p, const BlockArgs &a, hipStream_t st) {
    if (p.layout == 0 && p.pipe) {
        hipLaunchKernelGGL((k_layout0<ELEM, MODE, XBF16, true, 8>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
        return (int)hipGetLastError();
    }
    if constexpr ((MODE == kToken && XBF16) || MODE == kDequant) {
        if (p.layout == 0 && p.tail) return launch_layout0_tail<ELEM, MODE>(p, a, st);   // whole row groups + split tail
    }
    if constexpr ((MODE == kToken && XBF16) || MODE == kDequant) {
        if (p.layout == 0 && p.seq13 && !p.pipe && p.G < 65536u) {
            if (p.split == 2) launch_layout0p<ELEM, 4, MODE>(p, a, st);
            else if (p.split == 4) launch_layout0p<ELEM, 2, MODE>(p, a, st);
            else launch_layout0p<ELEM, 8, MODE>(p, a, st);
            return (int)hipGetLastError();
        }
    }
    if constexpr ((MODE == kToken && XBF16) || MODE == kDequant) {
        if (p.layout == 0 && p.seq13 && !p.pipe) {
            if (p.split == 2)
                hipLaunchKernelGGL((k_layout0<ELEM, MODE, XBF16, false, 4, kPeekSeq>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
            else if (p.split == 4)
                hipLaunchKernelGGL((k_layout0<ELEM, MODE, XBF16, false, 2, kPeekSeq>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
            else
                hipLaunchKernelGGL((k_layout0<ELEM, MODE, XBF16, false, 8, kPeekSeq>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
            return (int)hipGetLastError();
        }
    }
    if (p.layout == 0 && p.split == 2 && (MODE == kToken || MODE == kF32))
        hipLaunchKernelGGL((k_layout0<ELEM, MODE, XBF16, false, 4>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
    else if (p.layout == 0 && p.split == 4 && (MODE == kToken || MODE == kF32))
        hipLaunchKernelGGL((k_layout0<ELEM, MODE, XBF16, false, 2>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
    else if (p.layout == 0)
        hipLaunchKernelGGL((k_layout0<ELEM, MODE, XBF16, false, 8>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
    else if (p.layout == 1 && p.split)
        return launch_layout1s<ELEM, MODE, XBF16>(p, a, st);
    else if constexpr (MODE != kRowIndex)
        hipLaunchKernelGGL((k_layout1<ELEM, MODE, XBF16>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
    else
        return -1;
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Layout 0, token path for NT activation vectors at once (small batches: a few tokens, speculative drafts).  Tiles,
// stream staging and the raw-row ring are those of k_layout0's single-round path with one half-wave per block (NR = 8);
// every decoded weight pair goes through NT v_dot2, one per vector, so the NT products share one decode and one read
// of the matrix.  x is BF16 [NT][K16], y BF16 [NT][M]; each vector's sums follow the single-vector kernel's order
// exactly (lane order within a step, steps in order, the transposed half-wave reduction, column blocks ascending), so
// y[t] is bit-identical to a single-vector launch on x[t].
template <int ELEM, int NT, class Tab>
__device__ __forceinline__ void row0_batch(Seq<ELEM> &S, const Tab &s, const uint4 &rw, const XRegs<true> (&x)[NT],
                                           float (&sum)[NT]) {
#pragma unroll
    for (int t = 0; t < NT; t++) sum[t] = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t s0 = S.s;
        const uint32_t *wp0 = S.wp;
        uint32_t e1, e2;
        if (__builtin_expect(__any(S.fast_quad(s, e1, e2) >= kSeqSlowTest), 0)) {
            S.s = s0;
            S.wp = wp0;
            S.reload();
            S.slow_quad(s, e1, e2);
        }
        const uint32_t rk = u4_get(rw, k);
        const uint32_t p0 = perm(e1, rk, kSelPair0), p1 = perm(e2, rk, kSelPair2);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            sum[t] = dot2_bf16(p0, x[t].b[2 * k], sum[t]);
            sum[t] = dot2_bf16(p1, x[t].b[2 * k + 1], sum[t]);
            asm volatile("" : "+v"(sum[t]));
        }
    }
}

// The eight rows of one block for NT vectors; `global`: the lane's stream read from memory (a round that does not fit
// its LDS region), raw rows loaded as needed.  Returns, per vector, the row sums reduced as in rowsN (lane 4r: row r).
template <int ELEM, int NT, bool GLOBAL, class Tab>
__device__ __forceinline__ void rows_batch(const Tab &s, const uint32_t *lane, const BlockArgs &a, const Shape &f,
                                           const XRegs<true> (&x)[NT], uint4 ring[kRing0], const Coord0 &c, uint32_t L,
                                           float (&out)[NT]) {
    Seq<ELEM> S;
    S.init_at(lane, 0u);
    float acc[NT][8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        float sum[NT];
        if constexpr (GLOBAL) {
            row0_batch<ELEM, NT>(S, s, raw_row<ELEM>(a.low, f, c, r), x, sum);
        } else {
            row0_batch<ELEM, NT>(S, s, ring[r % kRing0], x, sum);
            if (r + kRing0 < 8) ring[r % kRing0] = raw_row<ELEM>(a.low, f, c, r + kRing0);
        }
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t][r] = c.col_ok ? sum[t] : 0.f;
    }
#pragma unroll
    for (int t = 0; t < NT; t++) out[t] = reduce8_transposed(acc[t], L);
}

// The first inputs come as the eight preloaded scalar arguments of k_layout0p (the table argument: the table this
// kernel stages); pk = G | H << 16 | stride / 16 << 22.
template <int ELEM, int NT, int PEEK = kPeek>
__global__ void __launch_bounds__(1024) k_layout0_batch(const uint8_t *__restrict__ data,
                                                        const uint32_t *__restrict__ bases,
                                                        const uint32_t *__restrict__ tab, uint32_t M, uint32_t K,
                                                        uint32_t pk, const uint8_t *__restrict__ hdr,
                                                        const void *__restrict__ xp, BlockArgs a) {
    __shared__ LutT<PEEK> s;
    extern __shared__ uint32_t dyn[];
    take_preloaded(a, data, bases, tab, M, K, pk, hdr, xp);
    if (PEEK != kPeekSeq) a.lut = tab;
    a.G = pk & 0xFFFFu;
    const uint32_t tid = threadIdx.x, nth = ((pk >> 16) & 0x3Fu) * 32u, L = tid & 31, hw = tid >> 5, H = nth >> 5;
    const uint32_t cap = a.slot_words * H;                    // one region slot per half-wave (one block each)
    uint32_t *cur = dyn;
    float *part = (float *)(dyn + cap);                       // [G * 8 rows][CB][NT]
    const Shape f(a.M, a.K, 0);
    const uint32_t rg0 = blockIdx.x * a.G;
    const uint32_t ng = min(a.G, f.groups() - rg0);
    const uint32_t nt = ng * f.CB, tl = nt - 1u;
    const uint32_t B0 = rg0 * f.CB, nb = f.nb;
    const uint32_t mend = !a.stride && B0 + nt == nb ? matrix_end(a, nb) : 0u;
    const uint32_t t = hw;
    const Coord0 c = coord0(min(t, tl), rg0, f, L);
    const Region R = region_of(a, B0, B0 + min(H, nt), nb, mend, a.stride);
    TabStage<PEEK> Q;
    Q.issue(a, nth);
    const uint32_t n = a.hdr[(uint64_t)c.b * kHdrBytes + L], base = block_base(a, c.b);
    Bulk Bk;
    bulk_issue(Bk, a.data, R, tid, nth);
    XRegs<true> x[NT];
#pragma unroll
    for (int v = 0; v < NT; v++) load_x16<true>(x[v], (const uint16_t *)a.x + (uint64_t)v * f.K16, c.col0, c.col_ok);
    // fp8: the scale and bias of this thread's first output (row rg0 * 8 + tid / NT), requested after the streams
    // (their pointers are read from the argument struct, and the wait for that read must not hold back the copy)
    float fin_scale = 1.f, fin_bias = 0.f;
    if (ELEM == kElemFp8 && tid < ng * kRows0 * NT && rg0 * kRows0 + tid / NT < a.M) {
        if (a.scale) fin_scale = a.scale[rg0 * kRows0 + tid / NT];
        if (a.bias) fin_bias = __uint_as_float((uint32_t)a.bias[rg0 * kRows0 + tid / NT] << 16);
    }
    Q.commit(s, nth);
    Q.finish(s, a, nth);
    const bool fits = R.n16 * 4u <= cap;
    if (fits) bulk_commit(Bk, cur, R, tid, nth);
    uint4 ring[kRing0];                                         // once this wave's stream chunks are in
#pragma unroll
    for (int r = 0; r < kRing0; r++) ring[r] = raw_row<ELEM>(a.low, f, c, r);
    __syncthreads();
    if (t < nt) {
        const uint32_t start = c.col_ok ? half_scan_incl(n, L) - n : 0u;
        float v[NT];
        if (fits) rows_batch<ELEM, NT, false>(s, cur + ((base - R.lo16) >> 2) + start, a, f, x, ring, c, L, v);
        else rows_batch<ELEM, NT, true>(s, (const uint32_t *)(a.data + base) + start, a, f, x, ring, c, L, v);
        if ((L & 3u) == 0) {
#pragma unroll
            for (int u = 0; u < NT; u++) part[((c.g * kRows0 + (L >> 2)) * f.CB + c.cb) * NT + u] = v[u];
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < ng * kRows0 * NT; i += nth) {
        const uint32_t u = i % NT, rr = i / NT, row = rg0 * kRows0 + rr;
        if (row >= a.M) continue;
        float acc = 0.f;
        for (uint32_t cb = 0; cb < f.CB; cb++) acc += part[(rr * f.CB + cb) * NT + u];
        const bool first = ELEM == kElemFp8 && i == threadIdx.x;
        if (a.scale) acc *= first ? fin_scale : a.scale[row];
        if (a.bias) acc += first ? fin_bias : __uint_as_float((uint32_t)a.bias[row] << 16);
        ((uint16_t *)a.out)[(uint64_t)u * a.M + row] = (uint16_t)f32_to_bf16_rne(acc);
    }
}

template <int ELEM, int PEEK>
static int launch_batch_t(const LaunchPlan &p, const BlockArgs &a, uint32_t ntok, hipStream_t st) {
    const dim3 g(p.grid), b(p.threads);
    const uint32_t pk = p.G | ((p.threads / 32u) << 16) | ((a.stride >> 4) << 22);
    const uint32_t *tab = PEEK == kPeekSeq ? a.seq : a.lut;
#define NWC_B_PRELOAD a.data, a.bases, tab, a.M, a.K, pk, a.hdr, a.x, a
    switch (ntok) {
    case 2: hipLaunchKernelGGL((k_layout0_batch<ELEM, 2, PEEK>), g, b, p.lds, st, NWC_B_PRELOAD); break;
    case 3: hipLaunchKernelGGL((k_layout0_batch<ELEM, 3, PEEK>), g, b, p.lds, st, NWC_B_PRELOAD); break;
    case 4: hipLaunchKernelGGL((k_layout0_batch<ELEM, 4, PEEK>), g, b, p.lds, st, NWC_B_PRELOAD); break;
    default: return -1;
    }
#undef NWC_B_PRELOAD
    return (int)hipGetLastError();
}

int launch_layout0_batch(const LaunchPlan &p, int elem_t, const BlockArgs &a, uint32_t ntok, hipStream_t st) {
    if (elem_t == kElemFp8)
        return p.seq13 ? launch_batch_t<kElemFp8, kPeekSeq>(p, a, ntok, st) : launch_batch_t<kElemFp8, kPeek>(p, a, ntok, st);
    return p.seq13 ? launch_batch_t<kElemBf16, kPeekSeq>(p, a, ntok, st) : launch_batch_t<kElemBf16, kPeek>(p, a, ntok, st);
}

int launch_prefix(const LaunchPlan &p, int elem_t, int mode, bool xbf16, const BlockArgs &a, hipStream_t st) {
    if (elem_t == kElemFp8) {
        if (mode == kDequant) return launch_prefix_t<kElemFp8, kDequant, true>(p, a, st);
        if (mode == kRowIndex) return launch_prefix_t<kElemFp8, kRowIndex, true>(p, a, st);
        if (mode == kF32) return launch_prefix_t<kElemFp8, kF32, false>(p, a, st);
        return xbf16 ? launch_prefix_t<kElemFp8, kToken, true>(p, a, st) : launch_prefix_t<kElemFp8, kToken, false>(p, a, st);
    }
    if (mode == kDequant) return launch_prefix_t<kElemBf16, kDequant, true>(p, a, st);
    if (mode == kRowIndex) return launch_prefix_t<kElemBf16, kRowIndex, true>(p, a, st);
    if (mode == kF32) return launch_prefix_t<kElemBf16, kF32, false>(p, a, st);
    return xbf16 ? launch_prefix_t<kElemBf16, kToken, true>(p, a, st) : launch_prefix_t<kElemBf16, kToken, false>(p, a, st);
}

int launch_gather_prefix(int layout, int elem_t, const GatherArgs &a, hipStream_t st) {
    const uint32_t per = 8;                                        // (id, column block) items per 256-thread workgroup
    const uint64_t items = (uint64_t)a.n_ids * Shape(a.M, a.K, layout).CB;
    const dim3 grid((uint32_t)((items + per - 1) / per));
    const size_t lds = (size_t)per * a.slot_words * 4;
    if (layout == 0) {
        if (elem_t == kElemFp8) hipLaunchKernelGGL(k_gather0<kElemFp8>, grid, dim3(256), lds, st, a);
        else hipLaunchKernelGGL(k_gather0<kElemBf16>, grid, dim3(256), lds, st, a);
    } else {
        if (elem_t == kElemFp8) hipLaunchKernelGGL(k_gather1<kElemFp8>, grid, dim3(256), lds, st, a);
        else hipLaunchKernelGGL(k_gather1<kElemBf16>, grid, dim3(256), lds, st, a);
    }
    return (int)hipGetLastError();
}

// Layout-0 row gather with the row index (nwc_gather_xindex): one half-wave per (id, column block), as k_gather0, but
// the cursor starts at the row pair that holds the row (the index's bit position of row 2j, j = (row % 8) / 2), so a
// half-wave decodes one or two rows (four or eight steps) instead of up to eight, with the token path's cursor and
// table (13-bit with `seq`, else the stored LUT re-encoded).  Out-of-range ids leave their output rows untouched.
template <int ELEM, int PEEK>
__global__ void __launch_bounds__(256) k_gather0x(GatherArgs a, const uint16_t *__restrict__ aux,
                                                 const uint32_t *__restrict__ seq) {
    __shared__ LutT<PEEK> s;
    extern __shared__ uint32_t dyn[];
    BlockArgs ta{};
    ta.lut = a.lut;
    ta.seq = seq;
    TabStage<PEEK> Q;
    Q.issue(ta);
    const uint32_t L = threadIdx.x & 31, hw = threadIdx.x >> 5;
    uint32_t *slot = dyn + hw * a.slot_words;
    const Shape f(a.M, a.K, 0);
    const uint32_t item = blockIdx.x * (blockDim.x >> 5) + hw, id = item / f.CB, cb = item - id * f.CB;
    Q.commit(s);
    Q.finish(s, ta);
    __syncthreads();                                              // every thread stages the table first
    if (id >= a.n_ids) return;
    const int64_t R = a.ids[id];
    if (R < 0 || R >= (int64_t)a.M) return;
    const uint32_t rb = (uint32_t)R / kRows0, rr = (uint32_t)R % kRows0;
    const uint32_t b = rb * f.CB + cb, col0 = cb * kCols + L * 16;
    const bool col_ok = col0 < f.K16;
    const LaneSpan sp = lane_span(a.hdr, b, L);
    const uint32_t base = a.bases[b];
    const uint4 raw = raw_row0<ELEM>(a.low, f, (uint32_t)R, col0, col_ok);
    const uint32_t P = rr >= 2u ? aux[((uint64_t)b * kRowIndexSplits + (rr >> 1) - 1u) * kLanes + L] : 0u;
    uint32_t sh;
    const bool staged = stage_block(slot, a.slot_words, a.data, base, sp.total, L, sh);
    const uint32_t *words = staged ? (const uint32_t *)slot + sh + sp.start : (const uint32_t *)(a.data + base) + sp.start;
    Seq<ELEM> S;
    S.init_at(words, P);
    const XRegs<true> xnone{};
    uint32_t pw[8];
    if (rr & 1u) row0<ELEM, kDequant, true>(S, s, raw, xnone, pw);    // the pair's first row, decoded past
    row0<ELEM, kDequant, true>(S, s, raw, xnone, pw);
    if (col_ok) {
        uint4 *op = (uint4 *)(a.out + (uint64_t)id * f.K16 + col0);
        op[0] = make_uint4(pw[0], pw[1], pw[2], pw[3]);
        op[1] = make_uint4(pw[4], pw[5], pw[6], pw[7]);
    }
}

// Layout 1: four half-waves per (id, column block), each decoding a quarter of the block's super-chunks (4p .. 4p + 3)
// from the row index's bit position of super-chunk 4p: 16 steps on the chain instead of up to 64.  Lanes whose row
// r = L / 4 (or r + 8) is the wanted one store its eight columns of each super-chunk, as k_gather1 does.
template <int ELEM, int PEEK>
__global__ void __launch_bounds__(256) k_gather1x(GatherArgs a, const uint16_t *__restrict__ aux,
                                                 const uint32_t *__restrict__ seq) {
    __shared__ LutT<PEEK> s;
    extern __shared__ uint32_t dyn[];
    BlockArgs ta{};
    ta.lut = a.lut;
    ta.seq = seq;
    TabStage<PEEK> Q;
    Q.issue(ta);
    constexpr uint32_t RB = ELEM == kElemFp8 ? 8u : 16u;
    const uint32_t L = threadIdx.x & 31, r = L >> 2, q = L & 3, hw = threadIdx.x >> 5;
    uint32_t *slot = dyn + hw * a.slot_words;
    const Shape f(a.M, a.K, 1);
    const uint32_t item = blockIdx.x * (blockDim.x >> 5) + hw, pair = item >> 2, p = item & 3u;
    const uint32_t id = pair / f.CB, cb = pair - id * f.CB;
    Q.commit(s);
    Q.finish(s, ta);
    __syncthreads();                                              // every thread stages the table first
    if (id >= a.n_ids) return;
    const int64_t R = a.ids[id];
    if (R < 0 || R >= (int64_t)a.M) return;
    const uint32_t rb = (uint32_t)R / kRows12, rr = (uint32_t)R % kRows12;
    const uint32_t nsc = ((cb == f.CB - 1 ? f.nl : 32u) + 1) / 2, sc0 = 4u * p;
    if (sc0 >= nsc) return;
    const uint32_t ns = min(4u, nsc - sc0), b = rb * f.CB + cb;
    const bool mine = (rr & 7u) == r, upper = rr >= 8;
    const uint8_t *rp = a.low + ((uint64_t)(rb * f.spr + cb * 16 + sc0) * kLanes + L) * RB;
    const LaneSpan sp = lane_span(a.hdr, b, L);
    const uint32_t base = a.bases[b];
    const uint32_t P = p ? aux[((uint64_t)b * kRowIndexSplits + p - 1u) * kLanes + L] : 0u;
    uint32_t sh;
    const bool staged = stage_block(slot, a.slot_words, a.data, base, sp.total, L, sh);
    const uint32_t *words = staged ? (const uint32_t *)slot + sh + sp.start : (const uint32_t *)(a.data + base) + sp.start;
    Seq<ELEM> S;
    S.init_at(words, P);
    uint16_t *o = a.out + (uint64_t)id * f.K16;
    for (uint32_t i = 0; i < ns; i++) {
        const uint4 raw = raw_slot1<ELEM>(rp + (uint64_t)i * kLanes * RB);
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t s0 = S.s;
            const uint32_t *wp0 = S.wp;
            uint32_t e1, e2;
            if (__builtin_expect(__any(S.fast_quad(s, e1, e2) >= kSeqSlowTest), 0)) {
                S.s = s0;
                S.wp = wp0;
                S.reload();
                S.slow_quad(s, e1, e2);
            }
            const uint32_t rk = u4_get(raw, k);
            v[k] = upper ? perm(e2, rk, kSelPair2) : perm(e1, rk, kSelPair0);
        }
        const uint32_t kc = cb * kCols + (sc0 + i) * 32 + 8 * q;
        if (mine && kc < f.K16) *(uint4 *)(o + kc) = make_uint4(v[0], v[1], v[2], v[3]);
    }
}

int launch_gather0x(int layout, int elem_t, const GatherArgs &a, const uint16_t *aux, const uint32_t *seq, hipStream_t st) {
    const uint32_t per = 8;                                        // half-wave items per 256-thread workgroup
    const uint64_t items = (uint64_t)a.n_ids * Shape(a.M, a.K, layout).CB * (layout == 1 ? 4u : 1u);
    const dim3 grid((uint32_t)((items + per - 1) / per));
    const size_t lds = (size_t)per * a.slot_words * 4;
#define NWC_GX(K_, E, T) hipLaunchKernelGGL((K_<E, T>), grid, dim3(256), lds, st, a, aux, seq)
    const bool fp8 = elem_t == kElemFp8;
    if (layout == 1) {
        if (seq) { if (fp8) NWC_GX(k_gather1x, kElemFp8, kPeekSeq); else NWC_GX(k_gather1x, kElemBf16, kPeekSeq); }
        else { if (fp8) NWC_GX(k_gather1x, kElemFp8, kPeek); else NWC_GX(k_gather1x, kElemBf16, kPeek); }
    } else {
        if (seq) { if (fp8) NWC_GX(k_gather0x, kElemFp8, kPeekSeq); else NWC_GX(k_gather0x, kElemBf16, kPeekSeq); }
        else { if (fp8) NWC_GX(k_gather0x, kElemFp8, kPeek); else NWC_GX(k_gather0x, kElemBf16, kPeek); }
    }
#undef NWC_GX
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Prefill of a layout-0 matrix without a temporary BF16 copy: y[t] = W x[t] (+ bias, x scale) for T tokens.
// A workgroup of 16 waves owns a tile of 64 rows (8 row groups) and TT tokens.  For each column block it decodes its
// eight blocks into LDS as BF16 (wave 2j copies block j's streams; four half-waves then decode two rows each from the
// row index's start, as dequantization does; lanes past K16 store zeros) and multiplies that 64 x 512 tile with the
// activations of its TT tokens on the matrix cores: v_mfma_f32_16x16x32_bf16 with A = 16 rows x 32 columns of the tile
// (one ds_read_b128 per lane: row lane & 15, columns 8 (lane >> 4) .. +7) and B = the same 32 columns of 16 tokens' x
// (one 16-byte load per lane, two or four k-steps ahead), fp32 accumulators over the whole K.  Up to 256 tokens per
// tile: more would not fit the accumulators next to the decode's registers without spilling.  The weights are decoded
// once per token tile and nothing but y is written.
constexpr uint32_t kPfRows = 64;                                 // rows per tile
constexpr uint32_t kPfStride = 2u * kCols + 16u;                 // tile row stride in bytes: rows 4 banks apart
constexpr uint32_t kPfSlot = 480;                                // stream words per block slot

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

// waves of a TT-token tile: every wave covers the tile's 64 rows (four 16-row subtiles) and 16 tokens; TS waves along
// the tokens, KS along the column block's 16 k-steps (each wave NK of them), so every activation is loaded once per
// workgroup; the KS partial sums are added through LDS at the end
template <int TT> struct PfShape {
    static_assert(TT == 64 || TT == 128 || TT == 256, "64, 128 or 256 tokens per tile");
    static constexpr int TS = TT / 16, KS = 16 / TS, NK = 16 / KS;
    static constexpr int AHEAD = 2;                               // k-steps of activations in flight per wave
};

// A block's streams for its staging slot, two 16-byte chunks per lane of a wave (the slot holds kPfSlot words); the loads
// are unconditional, at addresses clamped into the block's range.  start: the lane's word offset in the block; sh: the
// block's offset in the slot; fits: whether the block fits the slot (else it decodes from global memory).
__device__ __forceinline__ void pf_stage_issue(const BlockArgs &a, uint32_t n, uint32_t base, uint32_t L, uint32_t lane,
                                               uint4 &v0, uint4 &v1, uint32_t &start, uint32_t &sh, bool &fits) {
    const uint32_t incl = half_scan_incl(n, L), total = __shfl(incl, 31, 32);
    start = incl - n;
    sh = (base & 15u) >> 2;
    const uint32_t need = sh + total + 3u;
    fits = need <= kPfSlot;
    const uint8_t *src = a.data + (base & ~15u);
    const uint32_t last = ((min(need, kPfSlot) - 1u) & ~3u) * 4u;     // bytes; inside the block's range
    v0 = *(const uint4 *)(src + min(16u * lane, last));
    v1 = *(const uint4 *)(src + min(16u * lane + 1024u, last));
}
__device__ __forceinline__ void pf_stage_commit(uint32_t *slot, uint32_t lane, const uint4 &v0, const uint4 &v1) {
    *(uint4 *)(slot + 4u * lane) = v0;
    if (4u * lane + 256u < kPfSlot) *(uint4 *)(slot + 4u * lane + 256u) = v1;
}

// two rows of a block for one lane from bit position P0 (separate call sites keep LDS and global reads apart)
template <int ELEM>
__device__ __forceinline__ void pf_rows(const LutLds13 &s, const uint32_t *lane, uint32_t P0, const uint4 (&raw)[2],
                                        const XRegs<true> &xnone, uint32_t (&pw)[2][8]) {
    Seq<ELEM> S;
    S.init_at(lane, P0);
#pragma unroll
    for (int r = 0; r < 2; r++) {
        row0<ELEM, kDequant, true>(S, s, raw[r], xnone, pw[r]);
        asm volatile("" : "+v"(pw[r][0]), "+v"(pw[r][7]));
    }
}

template <int ELEM, int TT>
__global__ void __launch_bounds__(1024) k_prefill0(PrefillArgs p) {
    using PS = PfShape<TT>;
    constexpr int WR = 4, TS = PS::TS, KS = PS::KS, NK = PS::NK, AH = PS::AHEAD;
    const BlockArgs &a = p.a;
    __shared__ LutT<kPeekSeq> s;
    extern __shared__ uint32_t dyn[];
    uint8_t *tile = (uint8_t *)dyn;
    uint32_t *slots = (uint32_t *)(tile + kPfRows * kPfStride);
    const uint32_t tid = threadIdx.x, L = tid & 31, lane = tid & 63, wv = tid >> 6, hw = tid >> 5;
    const Shape f(a.M, a.K, 0);
    const uint32_t rg0 = blockIdx.x * (kPfRows / kRows0), groups = f.groups(), CB = f.CB;
    // decode role: half-wave hw decodes rows 2q, 2q + 1 of tile block j (row group rg0 + j) of every column block; a
    // tile past the matrix's last row group decodes that group again into rows that are never stored.  Wave 2j stages
    // block j's streams.
    const uint32_t j = hw >> 2, q = hw & 3, jj = min(rg0 + j, groups - 1u) - rg0;
    const bool copier = (wv & 1u) == 0u;
    uint32_t *slot = slots + j * kPfSlot;
    // matrix-core role: the tile's 64 rows, tokens tok0 .. + 15, k-steps kg NK .. + NK - 1 of every column block
    const uint32_t ts = wv % TS, kg = wv / TS, tok0 = blockIdx.y * TT + 16u * ts;
    const uint32_t arow = (lane & 15u) * kPfStride + 16u * (lane >> 4);    // A: + 64 ks bytes, + 16 kPfStride i
    const uint16_t *xrow = p.xt + (uint64_t)min(tok0 + (lane & 15u), p.T - 1u) * f.K16;

    // Every load below is unconditional (clamped addresses, values masked or unused), so the compiler counts them
    // exactly and each wait covers only what it needs.  Column block cb + 1's streams, raw rows and row-index entry
    // are requested while cb decodes, and its first activations while cb's last products run.
    auto coord = [&](uint32_t cb) {
        Coord0 c = coord0(jj * CB + min(cb, CB - 1u), rg0, f, L);
        c.rb += 2u * q * f.K16;                                   // this half-wave's first row
        return c;
    };
    auto xload = [&](uint32_t cb, uint32_t i, bf16x8_t &dst) {   // k-step kg NK + i: columns + 8 (lane >> 4) .. + 7
        cb = min(cb, CB - 1u);
        const uint32_t col = cb * kCols + 32u * (kg * NK + i) + 8u * (lane >> 4);
        const uint32_t keep = col < f.K16 ? ~0u : 0u;             // 0 past K16 (its products are skipped or zero)
        const uint4 v = *(const uint4 *)(xrow + min(col, f.K16 - 8u));
        dst = __builtin_bit_cast(bf16x8_t, make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep));
    };

    TabStage<kPeekSeq> Q;
    Q.issue(a);
    // column block 0: staged now; column block 1's header byte and base requested
    Coord0 c = coord(0u);
    uint4 st0, st1;                                               // column block cb's stream chunks (two per lane)
    uint32_t start, sh;                                           // lane offset in the block, block offset in the slot
    bool fits;
    uint32_t base = a.bases[c.b];
    pf_stage_issue(a, a.hdr[(uint64_t)c.b * kHdrBytes + L], base, L, lane, st0, st1, start, sh, fits);
    uint4 raw[2] = {raw_row<ELEM>(a.low, f, c, 0u), raw_row<ELEM>(a.low, f, c, 1u)};
    uint32_t P0 = part_start(a, c.b, q, L);
    Coord0 c1 = coord(1u);
    uint32_t n1 = a.hdr[(uint64_t)c1.b * kHdrBytes + L], base1 = a.bases[c1.b];
    bf16x8_t xb[AH];
#pragma unroll
    for (int d = 0; d < AH; d++) xload((uint32_t)(d / NK), (uint32_t)(d % NK), xb[d]);
    Q.commit(s);
    if (copier && fits) pf_stage_commit(slot, lane, st0, st1);
    Q.finish(s, a);
    f32x4_t acc[WR];
#pragma unroll
    for (int i = 0; i < WR; i++) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const XRegs<true> xnone{};
    __syncthreads();                                              // table and column block 0's streams staged
    for (uint32_t cb = 0; cb < CB; cb++) {
        // ---- requests for column block cb + 1 (clamped past the last) ----
        uint4 sn0, sn1;
        uint32_t startn, shn;
        bool fitsn;
        pf_stage_issue(a, n1, base1, L, lane, sn0, sn1, startn, shn, fitsn);
        uint4 rawn[2] = {raw_row<ELEM>(a.low, f, c1, 0u), raw_row<ELEM>(a.low, f, c1, 1u)};
        const uint32_t P0n = part_start(a, c1.b, q, L);
        const Coord0 c2 = coord(cb + 2u);
        const uint32_t n2 = a.hdr[(uint64_t)c2.b * kHdrBytes + L], base2 = a.bases[c2.b];
        // ---- decode column block cb into the tile ----
        uint32_t pw[2][8];
        if (fits) pf_rows<ELEM>(s, slot + sh + start, P0, raw, xnone, pw);                      // LDS reads
        else pf_rows<ELEM>(s, (const uint32_t *)(a.data + base) + start, P0, raw, xnone, pw);      // global (rare)
#pragma unroll
        for (int r = 0; r < 2; r++) {
            uint4 *o = (uint4 *)(tile + (8u * j + 2u * q + r) * kPfStride + 32u * L);
            o[0] = c.col_ok ? make_uint4(pw[r][0], pw[r][1], pw[r][2], pw[r][3]) : make_uint4(0u, 0u, 0u, 0u);
            o[1] = c.col_ok ? make_uint4(pw[r][4], pw[r][5], pw[r][6], pw[r][7]) : make_uint4(0u, 0u, 0u, 0u);
        }
        __syncthreads();                                          // tile complete, slots free
        if (copier && fitsn) pf_stage_commit(slot, lane, sn0, sn1);   // column block cb + 1's streams
        // ---- products: this wave's NK k-steps of 32 columns (none past K16 in a last column block under 512) ----
        const uint32_t kn = min(16u, (f.K16 - cb * kCols + 31u) / 32u);
        auto wload = [&](int i, bf16x8_t (&dst)[WR]) {
#pragma unroll
            for (int r = 0; r < WR; r++)
                dst[r] = *(const bf16x8_t *)(tile + arow + 16u * kPfStride * r + 64u * (kg * NK + (uint32_t)i));
        };
        bf16x8_t wa[2][WR];
        wload(0, wa[0]);
#pragma unroll
        for (int i = 0; i < NK; i++) {
            if (i + 1 < NK) wload(i + 1, wa[(i + 1) & 1]);
            if (kg * NK + (uint32_t)i < kn) {
#pragma unroll
                for (int r = 0; r < WR; r++)
                    acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[i & 1][r], xb[i % AH], acc[r], 0, 0, 0);
            }
            // the ring runs on into the next column block
            const int nx = i + AH;
            xload(cb + (uint32_t)(nx / NK), (uint32_t)(nx % NK), xb[i % AH]);
        }
        __syncthreads();                                          // tile free, column block cb + 1's streams visible
        start = startn;
        sh = shn;
        fits = fitsn;
        base = base1;
        raw[0] = rawn[0];
        raw[1] = rawn[1];
        P0 = P0n;
        c = c1;
        c1 = c2;
        n1 = n2;
        base1 = base2;
    }
    // ---- the KS waves of a token group add their partial sums through LDS (the tile is free after the last barrier) ----
    if constexpr (KS > 1) {
        float *red = (float *)tile;                                // [wave][row subtile][4][64 lanes]
#pragma unroll
        for (int r = 0; r < WR; r++)
#pragma unroll
            for (int e = 0; e < 4; e++) red[((wv * WR + r) * 4 + e) * 64u + lane] = acc[r][e];
        __syncthreads();
        if (kg != 0) return;
#pragma unroll
        for (uint32_t g = 1; g < (uint32_t)KS; g++)
#pragma unroll
            for (int r = 0; r < WR; r++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[r][e] += red[(((g * TS + ts) * WR + r) * 4 + e) * 64u + lane];
    }
    // ---- y: lane holds rows 4 (lane >> 4) + e of each 16-row subtile, for token lane & 15 ----
    uint16_t *y = (uint16_t *)a.out;
    const uint32_t t = tok0 + (lane & 15u);
    if (t >= p.T) return;
#pragma unroll
    for (int r = 0; r < WR; r++) {
        const uint32_t m = rg0 * kRows0 + 16u * r + 4u * (lane >> 4);
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t me = min(m + (uint32_t)e, a.M - 1u);
            float v = acc[r][e];
            if (a.scale) v *= a.scale[me];
            if (a.bias) v += __uint_as_float((uint32_t)a.bias[me] << 16);
            h[e] = f32_to_bf16_rne(v);
        }
        uint16_t *o = y + (uint64_t)t * a.M + m;
        if ((a.M & 3u) == 0u && m + 3u < a.M) {
            *(uint2 *)o = make_uint2(h[0] | h[1] << 16, h[2] | h[3] << 16);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (m + (uint32_t)e < a.M) o[e] = (uint16_t)h[e];
        }
    }
}

int launch_prefill0(int elem_t, uint32_t tt, const PrefillArgs &p, hipStream_t st) {
    const Shape f(p.a.M, p.a.K, 0);
    const dim3 grid((f.groups() + kPfRows / kRows0 - 1u) / (kPfRows / kRows0), (p.T + tt - 1u) / tt), block(1024);
    const size_t lds = (size_t)kPfRows * kPfStride + 8u * kPfSlot * 4u;
#define NWC_PF(E, T_) hipLaunchKernelGGL((k_prefill0<E, T_>), grid, block, lds, st, p)
    if (elem_t == kElemFp8) {
        switch (tt) { case 64: NWC_PF(kElemFp8, 64); break; case 128: NWC_PF(kElemFp8, 128); break;
                      default: NWC_PF(kElemFp8, 256); break; }
    } else {
        switch (tt) { case 64: NWC_PF(kElemBf16, 64); break; case 128: NWC_PF(kElemBf16, 128); break;
                      default: NWC_PF(kElemBf16, 256); break; }
    }
#undef NWC_PF
    return (int)hipGetLastError();
}

}  // namespace nwc
