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
// Loads are unconditional and unmasked: rows past M and columns past K16 read row 0 / column 0 instead, so a loop
// that issues them keeps static wait counts and no select has to wait for the data.  Their products are garbage and
// are dropped: sums of lanes past K16 are zeroed (col_ok selects), rows past M are never stored.
template <int ELEM>
__device__ __forceinline__ uint4 raw_row0(const uint8_t *__restrict__ low, const Shape &f, uint32_t row, uint32_t col0, bool col_ok) {
    const bool ok = row < f.M && col_ok;
    const uint64_t r = ok ? row : 0u, c = ok ? col0 : 0u;
    if (ELEM == kElemFp8) return expand_nibbles(ldnt2(low + r * (f.K16 / 2) + c / 2));
    return ldnt4(low + r * f.K16 + c);
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
    return c;
}

// Weights of one window step for the accumulator / dequant output.
template <int MODE, bool XBF16>
__device__ __forceinline__ void use_quad(uint32_t e1, uint32_t e2, uint32_t rk, int k, const XRegs<XBF16> &x, float &sum,
                                         uint32_t pw[8]) {
    if constexpr (MODE == kDequant) {
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

// The eight rows of one layout-0 block for one lane, decoded from its LDS slot with all raw-plane rows already
// requested.  Returns the row sums reduced over the half-wave (lane 4r holds row r) or, for dequantization, stores
// the rows.  Fully unrolled: every row's raw bytes live in their own registers.
template <int ELEM, int MODE, bool XBF16>
__device__ __forceinline__ float rows0(const LutLds &s, const uint32_t *words, const BlockArgs &a, const Shape &f,
                                       const XRegs<XBF16> &x, const uint4 raw[8], const Coord0 &c, uint32_t L) {
    Window<ELEM, const uint32_t *> W;
    W.init(words);
    float acc[8];
#pragma unroll
    for (int r = 0; r < (int)kRows0; r++) {
        float sum = 0.f;
        uint32_t pw[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t e1, e2;
            W.quad(s, e1, e2);
            use_quad<MODE, XBF16>(e1, e2, u4_get(raw[r], k), k, x, sum, pw);
            // consume each step's weights before the next decode step (otherwise the compiler sinks every dot
            // product to the end of the unrolled block and keeps all decoded words live)
            if (MODE == kDequant) asm volatile("" : "+v"(pw[2 * k]), "+v"(pw[2 * k + 1]));
            else asm volatile("" : "+v"(sum));
        }
        if (MODE == kDequant) store_row0<MODE>(a, f, c.row0 + r, c.col0, c.col_ok, pw);
        else acc[r] = c.col_ok ? sum : 0.f;
    }
    return MODE == kDequant ? 0.f : reduce8_transposed(acc, L);
}

// The same for a block whose streams do not fit the LDS slot: decoded straight from global memory with a rolled row
// loop and its own raw loads (compact code; such blocks are rare, e.g. near-uniform exponent distributions).  Lanes
// past K16 have empty streams; the callers point them at the block's first word, since decoding zero bits walks up
// to 96 words (all escapes), which stays inside a block too large for the slot (>= 475 words).
template <int ELEM, int MODE, bool XBF16>
__device__ __forceinline__ float rows0_global(const LutLds &s, const uint32_t *words, const BlockArgs &a, const Shape &f,
                                              const XRegs<XBF16> &x, const Coord0 &c, uint32_t L) {
    Window<ELEM, const uint32_t *> W;
    W.init(words);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int r = 0; r < (int)kRows0; r++) {
        const uint4 cur = raw_row0<ELEM>(a.low, f, c.row0 + r, c.col0, c.col_ok);
        float sum = 0.f;
        uint32_t pw[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t e1, e2;
            W.quad(s, e1, e2);
            use_quad<MODE, XBF16>(e1, e2, u4_get(cur, k), k, x, sum, pw);
        }
        if (MODE == kDequant) {
            store_row0<MODE>(a, f, c.row0 + r, c.col0, c.col_ok, pw);
        } else {
#pragma unroll
            for (int i = 0; i < (int)kRows0 - 1; i++) acc[i] = acc[i + 1];    // rotation: at the end acc[i] = row i
            acc[kRows0 - 1] = c.col_ok ? sum : 0.f;
        }
    }
    return MODE == kDequant ? 0.f : reduce8_transposed(acc, L);
}

// Layout 0, one block per half-wave (tile of at most one block per half; also the fallback when LDS allows no
// second slot).  Everything a block needs is requested before the table is staged.
template <int ELEM, int MODE, bool XBF16>
__global__ void __launch_bounds__(1024) k_layout0(BlockArgs a) {
    __shared__ LutLds s;
    extern __shared__ uint32_t dyn[];
    const uint32_t tid = threadIdx.x, L = tid & 31;
    const uint32_t hw = tid >> 5, nhw = blockDim.x >> 5;
    uint32_t *slot = dyn + hw * a.slot_words;
    float *part = (float *)(dyn + nhw * a.slot_words);
    const Shape f(a.M, a.K, 0);
    const uint32_t rg0 = blockIdx.x * a.G;
    const uint32_t ng = min(a.G, f.groups() - rg0);
    const uint32_t nt = ng * f.CB;
    uint32_t t = hw;
    Coord0 c = coord0(min(t, nt - 1), rg0, f, L);
    uint32_t n = a.hdr[(uint64_t)c.b * kHdrBytes + L], base = a.bases[c.b];
    uint4 raw[8];
#pragma unroll
    for (int r = 0; r < (int)kRows0; r++) raw[r] = raw_row0<ELEM>(a.low, f, c.row0 + r, c.col0, c.col_ok);
    XRegs<XBF16> x;
    if (MODE != kDequant) load_x16<XBF16>(x, a.x, c.col0, c.col_ok);
    stage_lut(s, a.lut);
    while (t < nt) {
        const uint32_t incl = half_scan_incl(n, L);
        const uint32_t total = __shfl(incl, 31, 32), start = incl - n;
        uint32_t sh;
        float v;
        if (stage_block(slot, a.slot_words, a.data, base, total, L, sh))
            v = rows0<ELEM, MODE, XBF16>(s, slot + sh + start, a, f, x, raw, c, L);
        else
            v = rows0_global<ELEM, MODE, XBF16>(s, (const uint32_t *)(a.data + base) + (c.col_ok ? start : 0u), a, f, x, c, L);
        if (MODE != kDequant && (L & 3) == 0) part[(c.g * kRows0 + (L >> 2)) * f.CB + c.cb] = v;
        t += nhw;
        if (t >= nt) break;
        __builtin_amdgcn_wave_barrier();                        // the slot is overwritten by the next block
        c = coord0(t, rg0, f, L);
        n = a.hdr[(uint64_t)c.b * kHdrBytes + L];
        base = a.bases[c.b];
#pragma unroll
        for (int r = 0; r < (int)kRows0; r++) raw[r] = raw_row0<ELEM>(a.low, f, c.row0 + r, c.col0, c.col_ok);
        if (MODE != kDequant) load_x16<XBF16>(x, a.x, c.col0, c.col_ok);
    }
    if (MODE != kDequant) finish_rows<MODE>(a, part, rg0 * kRows0, ng * kRows0, f.CB);
}

// A block's stream words copied ahead: four 16-byte loads per lane cover a 512-word slot (lanes past the block
// re-read its last chunk, so the count is fixed), written to LDS once the slot is free.
struct Ahead {
    u32x4_t v0, v1, v2, v3;     // native vectors: HIP's uint4 struct copies would go through a stack object
    uint32_t need, sh;
    bool fits;
};
__device__ __forceinline__ void ahead_issue(Ahead &A, const uint8_t *__restrict__ data, uint32_t base, uint32_t total,
                                            uint32_t L, uint32_t slot_words) {
    const uint8_t *p = data + (base & ~15u);
    A.sh = (base & 15u) >> 2;
    A.need = A.sh + total + 3;
    A.fits = A.need <= slot_words;
    const uint32_t last = (min(A.need, slot_words) - 1u) & ~3u;
    A.v0 = *(const u32x4_t *)(p + 4u * min(L * 4u, last));
    A.v1 = *(const u32x4_t *)(p + 4u * min(L * 4u + 128u, last));
    A.v2 = *(const u32x4_t *)(p + 4u * min(L * 4u + 256u, last));
    A.v3 = *(const u32x4_t *)(p + 4u * min(L * 4u + 384u, last));
}
__device__ __forceinline__ void ahead_commit(const Ahead &A, uint32_t *slot, uint32_t L) {
    if (!A.fits) return;
    const uint32_t i = L * 4u;
    if (i < A.need) *(u32x4_t *)(slot + i) = A.v0;
    if (i + 128u < A.need) *(u32x4_t *)(slot + i + 128u) = A.v1;
    if (i + 256u < A.need) *(u32x4_t *)(slot + i + 256u) = A.v2;
    if (i + 384u < A.need) *(u32x4_t *)(slot + i + 384u) = A.v3;
}

// Inputs of the next block, requested half a block ahead of their use.
template <bool XBF16>
struct Next0 {
    Ahead A;                    // stream words for its LDS slot
    XRegs<XBF16> x;             // activations
    uint32_t start;             // lane's first word inside the block
};

template <int ELEM, int MODE, bool XBF16>
__device__ __forceinline__ void next_issue(Next0<XBF16> &N, const BlockArgs &a, const Coord0 &nx, uint32_t n_n, uint32_t base_n,
                                           uint32_t L) {
    const uint32_t incl = half_scan_incl(n_n, L);
    N.start = incl - n_n;
    ahead_issue(N.A, a.data, base_n, __shfl(incl, 31, 32), L, a.slot_words);
    if (MODE != kDequant) load_x16<XBF16>(N.x, a.x, nx.col0, nx.col_ok);
}

// rows0 for the pipelined kernel: the raw-plane rows go through a ring of four registers (row r + 4 of this block is
// requested when row r is done, then rows 0-3 of the next block), and the next block's stream words and activations
// are requested at row 4.  Register cost of the look-ahead: 16 (ring) + 16 (stream) + activations.
template <int ELEM, int MODE, bool XBF16>
__device__ __forceinline__ float rows0_ring(const LutLds &s, const uint32_t *words, const BlockArgs &a, const Shape &f,
                                            const XRegs<XBF16> &x, uint4 ring[4], const Coord0 &c, const Coord0 &nx,
                                            uint32_t n_n, uint32_t base_n, Next0<XBF16> &N, uint32_t L) {
    Window<ELEM, const uint32_t *> W;
    W.init(words);
    float acc[8];
#pragma unroll
    for (int r = 0; r < (int)kRows0; r++) {
        if (r == 4) next_issue<ELEM, MODE, XBF16>(N, a, nx, n_n, base_n, L);
        float sum = 0.f;
        uint32_t pw[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t e1, e2;
            W.quad(s, e1, e2);
            use_quad<MODE, XBF16>(e1, e2, u4_get(ring[r & 3], k), k, x, sum, pw);
            if (MODE == kDequant) asm volatile("" : "+v"(pw[2 * k]), "+v"(pw[2 * k + 1]));
            else asm volatile("" : "+v"(sum));
        }
        ring[r & 3] = r < 4 ? raw_row0<ELEM>(a.low, f, c.row0 + r + 4, c.col0, c.col_ok)
                            : raw_row0<ELEM>(a.low, f, nx.row0 + r - 4, nx.col0, nx.col_ok);
        if (MODE == kDequant) store_row0<MODE>(a, f, c.row0 + r, c.col0, c.col_ok, pw);
        else acc[r] = c.col_ok ? sum : 0.f;
    }
    return MODE == kDequant ? 0.f : reduce8_transposed(acc, L);
}

// Layout 0, several blocks per half-wave, software-pipelined over two LDS slots per half: while block t decodes from
// one slot, the stream words, raw rows and activations of block t + H (H = half-waves of the workgroup) are in flight
// and the header and base of block t + 2H are read, so after the first block no step waits on global memory.
template <int ELEM, int MODE, bool XBF16>
__global__ void __launch_bounds__(1024) k_layout0_pipe(BlockArgs a) {
    __shared__ LutLds s;
    extern __shared__ uint32_t dyn[];
    const uint32_t tid = threadIdx.x, L = tid & 31;
    const uint32_t hw = tid >> 5, nhw = blockDim.x >> 5;
    uint32_t *cur = dyn + hw * 2u * a.slot_words, *nxt = cur + a.slot_words;
    float *part = (float *)(dyn + nhw * 2u * a.slot_words);
    const Shape f(a.M, a.K, 0);
    const uint32_t rg0 = blockIdx.x * a.G;
    const uint32_t ng = min(a.G, f.groups() - rg0);
    const uint32_t nt = ng * f.CB, tl = nt - 1;               // look-ahead past the tile re-reads block tl
    uint32_t t = hw;
    Coord0 c = coord0(min(t, tl), rg0, f, L), cn = coord0(min(t + nhw, tl), rg0, f, L);
    const uint32_t n = a.hdr[(uint64_t)c.b * kHdrBytes + L], base = a.bases[c.b];
    uint32_t n_n = a.hdr[(uint64_t)cn.b * kHdrBytes + L], base_n = a.bases[cn.b];
    uint4 ring[4];
#pragma unroll
    for (int r = 0; r < 4; r++) ring[r] = raw_row0<ELEM>(a.low, f, c.row0 + r, c.col0, c.col_ok);
    XRegs<XBF16> x;
    if (MODE != kDequant) load_x16<XBF16>(x, a.x, c.col0, c.col_ok);
    stage_lut(s, a.lut);
    if (t < nt) {
        const uint32_t incl = half_scan_incl(n, L);
        uint32_t start = incl - n, sh;
        bool fits = stage_block(cur, a.slot_words, a.data, base, __shfl(incl, 31, 32), L, sh);
        uint32_t base_c = base;
        for (;;) {
            const Coord0 cnn = coord0(min(t + 2u * nhw, tl), rg0, f, L);
            const uint32_t n_nn = a.hdr[(uint64_t)cnn.b * kHdrBytes + L], base_nn = a.bases[cnn.b];
            Next0<XBF16> N;
            float v;
            if (fits) {
                v = rows0_ring<ELEM, MODE, XBF16>(s, cur + sh + start, a, f, x, ring, c, cn, n_n, base_n, N, L);
            } else {
                next_issue<ELEM, MODE, XBF16>(N, a, cn, n_n, base_n, L);
                v = rows0_global<ELEM, MODE, XBF16>(s, (const uint32_t *)(a.data + base_c) + (c.col_ok ? start : 0u), a, f, x, c, L);
#pragma unroll
                for (int r = 0; r < 4; r++) ring[r] = raw_row0<ELEM>(a.low, f, cn.row0 + r, cn.col0, cn.col_ok);
            }
            if (MODE != kDequant && (L & 3) == 0) part[(c.g * kRows0 + (L >> 2)) * f.CB + c.cb] = v;
            t += nhw;
            if (t >= nt) break;
            ahead_commit(N.A, nxt, L);
            __builtin_amdgcn_wave_barrier();
            uint32_t *tmp = cur; cur = nxt; nxt = tmp;
            start = N.start; sh = N.A.sh; fits = N.A.fits; base_c = base_n;
            if (MODE != kDequant) x = N.x;
            c = cn;
            cn = cnn;
            n_n = n_nn;
            base_n = base_nn;
        }
    }
    if (MODE != kDequant) finish_rows<MODE>(a, part, rg0 * kRows0, ng * kRows0, f.CB);
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
    stage_lut(s, a.lut);
    constexpr uint32_t RB = ELEM == kElemFp8 ? 8u : 16u;           // raw bytes per lane and super-chunk
    const uint32_t tid = threadIdx.x, L = tid & 31, r = L >> 2, q = L & 3;
    const uint32_t hw = tid >> 5, nhw = blockDim.x >> 5;
    uint32_t *slot = dyn + hw * a.slot_words;
    float *part = (float *)(dyn + nhw * a.slot_words);
    const Shape f(a.M, a.K, 1);
    const uint32_t rg0 = blockIdx.x * a.G;
    const uint32_t ng = min(a.G, f.groups() - rg0);
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
    if (MODE != kDequant) finish_rows<MODE>(a, part, rg0 * kRows12, ng * kRows12, f.CB);
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
    stage_lut(s, a.lut);
    const uint32_t L = threadIdx.x & 31, hw = threadIdx.x >> 5;
    uint32_t *slot = dyn + hw * a.slot_words;
    const uint32_t id = blockIdx.x * (blockDim.x >> 5) + hw;
    if (id >= a.n_ids) return;
    const int64_t R = a.ids[id];
    if (R < 0 || R >= (int64_t)a.M) return;
    const Shape f(a.M, a.K, 0);
    const uint32_t rb = (uint32_t)R / kRows0, rr = (uint32_t)R % kRows0;
    uint16_t *o = a.out + (uint64_t)id * f.K16;
    for (uint32_t cb = 0; cb < f.CB; cb++) {
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
        __builtin_amdgcn_wave_barrier();                        // the slot is overwritten by the next block
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
    stage_lut(s, a.lut);
    constexpr uint32_t RB = ELEM == kElemFp8 ? 8u : 16u;
    const uint32_t L = threadIdx.x & 31, r = L >> 2, q = L & 3, hw = threadIdx.x >> 5;
    uint32_t *slot = dyn + hw * a.slot_words;
    const uint32_t id = blockIdx.x * (blockDim.x >> 5) + hw;
    if (id >= a.n_ids) return;
    const int64_t R = a.ids[id];
    if (R < 0 || R >= (int64_t)a.M) return;
    const Shape f(a.M, a.K, 1);
    const uint32_t rb = (uint32_t)R / kRows12, rr = (uint32_t)R % kRows12;
    const bool mine = (rr & 7u) == r, upper = rr >= 8;
    uint16_t *o = a.out + (uint64_t)id * f.K16;
    for (uint32_t cb = 0; cb < f.CB; cb++) {
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
        __builtin_amdgcn_wave_barrier();
    }
}

// ---------------------------------------------------------------------------------------------------------------
template <int ELEM, int MODE, bool XBF16>
static int launch_prefix_t(const LaunchPlan &p, const BlockArgs &a, hipStream_t st) {
    if (p.layout == 0 && p.pipe)
        hipLaunchKernelGGL((k_layout0_pipe<ELEM, MODE, XBF16>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
    else if (p.layout == 0)
        hipLaunchKernelGGL((k_layout0<ELEM, MODE, XBF16>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
    else
        hipLaunchKernelGGL((k_layout1<ELEM, MODE, XBF16>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
    return (int)hipGetLastError();
}

int launch_prefix(const LaunchPlan &p, int elem_t, int mode, bool xbf16, const BlockArgs &a, hipStream_t st) {
    if (elem_t == kElemFp8) {
        if (mode == kDequant) return launch_prefix_t<kElemFp8, kDequant, true>(p, a, st);
        if (mode == kF32) return launch_prefix_t<kElemFp8, kF32, false>(p, a, st);
        return xbf16 ? launch_prefix_t<kElemFp8, kToken, true>(p, a, st) : launch_prefix_t<kElemFp8, kToken, false>(p, a, st);
    }
    if (mode == kDequant) return launch_prefix_t<kElemBf16, kDequant, true>(p, a, st);
    if (mode == kF32) return launch_prefix_t<kElemBf16, kF32, false>(p, a, st);
    return xbf16 ? launch_prefix_t<kElemBf16, kToken, true>(p, a, st) : launch_prefix_t<kElemBf16, kToken, false>(p, a, st);
}

int launch_gather_prefix(int layout, int elem_t, const GatherArgs &a, hipStream_t st) {
    const uint32_t per = 8;                                        // ids per 256-thread workgroup (one per half-wave)
    const dim3 grid((a.n_ids + per - 1) / per);
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

}  // namespace nwc
