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
template <bool XBF16>
struct XRegs {
    uint32_t b[8];
    float f[16];
};

// ---------------------------------------------------------------------------------------------------------------
// Layout 0: lane L of block (rb, cb) owns columns cb*512 + 16L .. +15 of rows rb*8 .. rb*8+7, stream order row-major.
template <int ELEM>
__device__ __forceinline__ uint4 raw_row0(const uint8_t *__restrict__ low, const Shape &f, uint32_t row, uint32_t col0, bool col_ok) {
    if (row < f.M && col_ok) {
        if (ELEM == kElemFp8) return expand_nibbles(ldnt2(low + (uint64_t)row * (f.K16 / 2) + col0 / 2));
        return ldnt4(low + (uint64_t)row * f.K16 + col0);
    }
    return make_uint4(0u, 0u, 0u, 0u);
}

template <bool XBF16>
__device__ __forceinline__ void load_x16(XRegs<XBF16> &x, const void *xp, uint32_t col0, bool col_ok) {
    if (XBF16) {
        uint4 v0 = make_uint4(0, 0, 0, 0), v1 = v0;
        if (col_ok) { const uint4 *p = (const uint4 *)((const uint16_t *)xp + col0); v0 = p[0]; v1 = p[1]; }
        x.b[0] = v0.x; x.b[1] = v0.y; x.b[2] = v0.z; x.b[3] = v0.w; x.b[4] = v1.x; x.b[5] = v1.y; x.b[6] = v1.z; x.b[7] = v1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = col_ok ? ((const float4 *)((const float *)xp + col0))[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            x.f[4 * i] = v.x; x.f[4 * i + 1] = v.y; x.f[4 * i + 2] = v.z; x.f[4 * i + 3] = v.w;
        }
    }
}

// The eight rows of one layout-0 block for one lane (raw rows already requested).  Returns the block's row sums
// reduced over the half-wave (lane 4r holds row r) or, for dequantization, stores the rows.  Fully unrolled: every
// row's raw bytes live in their own registers, so the loop never waits on a load issued inside it.
template <int ELEM, int MODE, bool XBF16, typename P>
__device__ __forceinline__ float rows0(const LutLds &s, P words, const BlockArgs &a, const Shape &f, const XRegs<XBF16> &x,
                                       const uint4 raw[8], uint32_t row0, uint32_t col0, bool col_ok, uint32_t L) {
    Window<ELEM, P> W;
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
            const uint32_t rk = u4_get(raw[r], k);
            if (MODE == kDequant) {
                pw[2 * k] = perm(e1, rk, kSelPair0);
                pw[2 * k + 1] = perm(e2, rk, kSelPair2);
            } else if (XBF16) {
                sum = dot2_bf16(perm(e1, rk, kSelPair0), x.b[2 * k], sum);
                sum = dot2_bf16(perm(e2, rk, kSelPair2), x.b[2 * k + 1], sum);
            } else {
                sum = fmaf(__uint_as_float(perm(e1, rk, sel_f32(0, 5))), x.f[4 * k], sum);
                sum = fmaf(__uint_as_float(perm(e1, rk, sel_f32(1, 6))), x.f[4 * k + 1], sum);
                sum = fmaf(__uint_as_float(perm(e2, rk, sel_f32(2, 5))), x.f[4 * k + 2], sum);
                sum = fmaf(__uint_as_float(perm(e2, rk, sel_f32(3, 6))), x.f[4 * k + 3], sum);
            }
            // consume each step's weights before the next decode step (otherwise the compiler sinks every dot
            // product to the end of the unrolled block and keeps all 64 decoded words live)
            if (MODE == kDequant) asm volatile("" : "+v"(pw[2 * k]), "+v"(pw[2 * k + 1]));
            else asm volatile("" : "+v"(sum));
        }
        if (MODE == kDequant) {
            if (row0 + r < f.M && col_ok) {
                uint4 *o = (uint4 *)((uint16_t *)a.out + (uint64_t)(row0 + r) * f.K16 + col0);
                o[0] = make_uint4(pw[0], pw[1], pw[2], pw[3]);
                o[1] = make_uint4(pw[4], pw[5], pw[6], pw[7]);
            }
        } else {
            acc[r] = sum;
        }
    }
    return MODE == kDequant ? 0.f : reduce8_transposed(acc, L);
}

// The same for a block whose streams do not fit the LDS slot: decoded straight from global memory with a rolled row
// loop (compact code; such blocks are rare, e.g. near-uniform exponent distributions).
template <int ELEM, int MODE, bool XBF16>
__device__ __noinline__ float rows0_global(const LutLds &s, const uint32_t *words, const BlockArgs &a, const Shape &f,
                                           uint32_t row0, uint32_t col0, bool col_ok, uint32_t L) {
    XRegs<XBF16> x;
    if (MODE != kDequant) load_x16<XBF16>(x, a.x, col0, col_ok);
    Window<ELEM, const uint32_t *> W;
    W.init(words);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int r = 0; r < (int)kRows0; r++) {
        const uint4 cur = raw_row0<ELEM>(a.low, f, row0 + r, col0, col_ok);
        float sum = 0.f;
        uint32_t pw[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t e1, e2;
            W.quad(s, e1, e2);
            const uint32_t rk = u4_get(cur, k);
            if (MODE == kDequant) {
                pw[2 * k] = perm(e1, rk, kSelPair0);
                pw[2 * k + 1] = perm(e2, rk, kSelPair2);
            } else if (XBF16) {
                sum = dot2_bf16(perm(e1, rk, kSelPair0), x.b[2 * k], sum);
                sum = dot2_bf16(perm(e2, rk, kSelPair2), x.b[2 * k + 1], sum);
            } else {
                sum = fmaf(__uint_as_float(perm(e1, rk, sel_f32(0, 5))), x.f[4 * k], sum);
                sum = fmaf(__uint_as_float(perm(e1, rk, sel_f32(1, 6))), x.f[4 * k + 1], sum);
                sum = fmaf(__uint_as_float(perm(e2, rk, sel_f32(2, 5))), x.f[4 * k + 2], sum);
                sum = fmaf(__uint_as_float(perm(e2, rk, sel_f32(3, 6))), x.f[4 * k + 3], sum);
            }
        }
        if (MODE == kDequant) {
            if (row0 + r < f.M && col_ok) {
                uint4 *o = (uint4 *)((uint16_t *)a.out + (uint64_t)(row0 + r) * f.K16 + col0);
                o[0] = make_uint4(pw[0], pw[1], pw[2], pw[3]);
                o[1] = make_uint4(pw[4], pw[5], pw[6], pw[7]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < (int)kRows0 - 1; i++) acc[i] = acc[i + 1];    // rotation: at the end acc[i] = row i
            acc[kRows0 - 1] = sum;
        }
    }
    return MODE == kDequant ? 0.f : reduce8_transposed(acc, L);
}

template <int ELEM, int MODE, bool XBF16>
__global__ void __launch_bounds__(1024) k_layout0(BlockArgs a) {
    __shared__ LutLds s;
    extern __shared__ uint32_t dyn[];
    stage_lut(s, a.lut);
    const uint32_t tid = threadIdx.x, L = tid & 31;
    const uint32_t hw = tid >> 5, nhw = blockDim.x >> 5;
    uint32_t *slot = dyn + hw * a.slot_words;
    float *part = (float *)(dyn + nhw * a.slot_words);
    const Shape f(a.M, a.K, 0);
    const uint32_t rg0 = blockIdx.x * a.G;
    const uint32_t ng = min(a.G, f.groups() - rg0);
    const uint32_t nt = ng * f.CB;

    for (uint32_t t = hw; t < nt; t += nhw) {
        const uint32_t g = t / f.CB, cb = t - g * f.CB, rb = rg0 + g, b = rb * f.CB + cb;
        const uint32_t row0 = rb * kRows0, col0 = cb * kCols + L * 16;
        const bool col_ok = col0 < f.K16;
        const LaneSpan sp = lane_span(a.hdr, b, L);
        const uint32_t base = a.bases[b];
        // all raw rows and the activations are requested before the stream copy; its wait covers them
        uint4 raw[8];
#pragma unroll
        for (int r = 0; r < (int)kRows0; r++) raw[r] = raw_row0<ELEM>(a.low, f, row0 + r, col0, col_ok);
        XRegs<XBF16> x;
        if (MODE != kDequant) load_x16<XBF16>(x, a.x, col0, col_ok);
        uint32_t sh;
        float v;
        if (stage_block(slot, a.slot_words, a.data, base, sp.total, L, sh))
            v = rows0<ELEM, MODE, XBF16>(s, (const uint32_t *)slot + sh + sp.start, a, f, x, raw, row0, col0, col_ok, L);
        else
            v = rows0_global<ELEM, MODE, XBF16>(s, (const uint32_t *)(a.data + base) + sp.start, a, f, row0, col0, col_ok, L);
        if (MODE != kDequant && (L & 3) == 0) part[(g * kRows0 + (L >> 2)) * f.CB + cb] = v;
        __builtin_amdgcn_wave_barrier();                        // the slot is overwritten by the next block
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
    accA += xor_f(accA, 1); accA += xor_f(accA, 2);            // the four lanes of a row pair
    accB += xor_f(accB, 1); accB += xor_f(accB, 2);
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
    if (p.layout == 0)
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
