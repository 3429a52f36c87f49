// kern_fixed.hip -- gfx950 kernels for layout 2 (format v11): fixed-width [sign | rank] nibbles, a raw plane and
// per-lane exception lists, in layout 1's 16 x 512 blocks and fragment order (docs/format.md section 4d).
//
// No bit window: per lane and 32-column super-chunk one 8-byte nibble load, one 16-byte raw load (fp8: three words
// per super-chunk pair) and one 16-byte activation load.  Eight ranks at a time go through v_perm_b32 against the
// 8-byte rank table held in two registers; signs come from bit 3 of the nibbles; BF16 pairs for v_dot2_f32_bf16
// are assembled with two more v_perm_b32.  Exceptions (rank 7, planes zero) are added after the super-chunks.
#include "nwc_device.h"
#include "nwc_launch.h"

namespace nwc {

struct RankTab { uint32_t T0, T1, U0, U1; };   // table byte of ranks 0..7; low-byte bit 7 of ranks 0..7 (fp8)

// 8 positions (one nibble word) -> the high bytes of positions 0..3 and 4..7 of the word, BF16 byte order
__device__ __forceinline__ void ranks8(const RankTab &t, uint32_t nw, uint32_t &h03, uint32_t &h47, uint32_t &l03, uint32_t &l47, bool fp8) {
    const uint32_t a = nw & 0x0F0F0F0Fu;                 // nibbles of positions 0, 2, 4, 6
    const uint32_t b = (nw >> 4) & 0x0F0F0F0Fu;          // positions 1, 3, 5, 7
    const uint32_t ra = a & 0x07070707u, rb = b & 0x07070707u;
    const uint32_t ha = perm(t.T1, t.T0, ra) | ((a << 4) & 0x80808080u);
    const uint32_t hb = perm(t.T1, t.T0, rb) | ((b << 4) & 0x80808080u);
    h03 = perm(hb, ha, 0x05010400u);
    h47 = perm(hb, ha, 0x07030602u);
    if (fp8) {
        const uint32_t la = perm(t.U1, t.U0, ra), lb = perm(t.U1, t.U0, rb);
        l03 = perm(lb, la, 0x05010400u);
        l47 = perm(lb, la, 0x07030602u);
    } else {
        l03 = l47 = 0u;
    }
}
// BF16 pairs of positions (0,1) and (2,3) of a 4-position group: [low0 | high0][low1 | high1]
constexpr uint32_t kSelLoHi01 = 0x05010400u;
constexpr uint32_t kSelLoHi23 = 0x07030602u;

// bits 12G .. 12G+11 of the 96-bit little-endian integer w2:w1:w0 (G a compile-time constant after unrolling)
__device__ __forceinline__ uint32_t bits12(uint32_t w0, uint32_t w1, uint32_t w2, int G) {
    const int bit = 12 * G, k = bit >> 5, sh = bit & 31;
    const uint32_t lo = k == 0 ? w0 : k == 1 ? w1 : w2, hi = k == 0 ? w1 : k == 1 ? w2 : 0u;
    return __builtin_amdgcn_alignbit(hi, lo, (uint32_t)sh) & 0xFFFu;
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
    const uint32_t e = (b >> 3) & 15u, m = b & 7u;
    const float v = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0.001953125f;
    return (b & 0x80u) ? -v : v;
}

template <int ELEM>
__device__ __forceinline__ float exc_value(const uint8_t *e) {
    if (ELEM == kElemFp8) return e4m3_to_f32(e[1]);
    return __uint_as_float(((uint32_t)e[1] | ((uint32_t)e[2] << 8)) << 16);
}

// fp8: 12-bit index (four 3-bit fields) -> the four fields, each shifted into bits 4..6 of its byte
struct MantLds { uint32_t m[kLutWords]; };
__device__ __forceinline__ void stage_mant(MantLds &s) {
    for (uint32_t i = threadIdx.x; i < kLutWords; i += blockDim.x)
        s.m[i] = ((i & 7u) << 4) | (((i >> 3) & 7u) << 12) | (((i >> 6) & 7u) << 20) | (((i >> 9) & 7u) << 28);
    __syncthreads();
}

// Decodes one super-chunk of a lane: p[k] = BF16 pair of row r (positions 4k, 4k+1), q[k] = pair of row r+8.
template <int ELEM, int G0>
__device__ __forceinline__ void decode_sc(const RankTab &t, const MantLds *ms, uint2 nib, uint4 raw, uint32_t c0, uint32_t c1, uint32_t c2,
                                          uint32_t p[4], uint32_t q[4]) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
        uint32_t h03, h47, l03, l47;
        ranks8(t, h ? nib.y : nib.x, h03, h47, l03, l47, ELEM == kElemFp8);
        uint32_t r0, r1;                                          // low bytes of positions 8h+0..3 and 8h+4..7
        if (ELEM == kElemFp8) {
            r0 = ms->m[bits12(c0, c1, c2, G0 + 2 * h)] | l03;
            r1 = ms->m[bits12(c0, c1, c2, G0 + 2 * h + 1)] | l47;
        } else {
            r0 = h ? raw.z : raw.x;
            r1 = h ? raw.w : raw.y;
        }
        p[2 * h] = perm(h03, r0, kSelLoHi01);
        q[2 * h] = perm(h03, r0, kSelLoHi23);
        p[2 * h + 1] = perm(h47, r1, kSelLoHi01);
        q[2 * h + 1] = perm(h47, r1, kSelLoHi23);
    }
}

// start of this lane's exception entries in block b (prefix over the half's counts)
__device__ __forceinline__ const uint8_t *exc_start(const BlockArgs &a, uint32_t b, uint32_t L, uint32_t esz, uint32_t &cnt) {
    cnt = a.hdr[(uint64_t)b * kHdrBytes + L];
    const uint32_t incl = half_scan_incl(cnt, L);
    return a.data + a.bases[b] + (uint64_t)(incl - cnt) * esz;
}

template <int ELEM, int MODE, bool XBF16>
__global__ void __launch_bounds__(1024) k_layout2(BlockArgs a) {
    __shared__ MantLds ms;
    extern __shared__ float part[];
    if (ELEM == kElemFp8) stage_mant(ms);
    const RankTab tab{a.lut[0], a.lut[1], a.lut[2], a.lut[3]};
    constexpr uint32_t esz = ELEM == kElemFp8 ? 2u : 3u;
    const uint32_t tid = threadIdx.x, L = tid & 31, r = L >> 2, q = L & 3;
    const uint32_t hw = tid >> 5, nhw = blockDim.x >> 5;
    const Shape f(a.M, a.K, 2);
    const uint8_t *rplane = a.low + f.nib2_bytes();
    const uint32_t rg0 = blockIdx.x * a.G;
    const uint32_t ng = min(a.G, f.groups() - rg0);
    const RowFinish fin = row_finish_load<MODE, ELEM == kElemFp8>(a, rg0 * kRows12, ng * kRows12);
    const uint32_t nt = ng * f.CB;

    for (uint32_t t = hw; t < nt; t += nhw) {
        const uint32_t g = t / f.CB, cb = t - g * f.CB, rb = rg0 + g, b = rb * f.CB + cb;
        const uint32_t row0 = rb * kRows12;
        const uint32_t nsc = ((cb == f.CB - 1 ? f.nl : 32u) + 1) / 2, slot0 = rb * f.spr + cb * 16;
        const uint8_t *np = a.low + ((uint64_t)slot0 * kLanes + L) * 8;
        const uint8_t *rp = ELEM == kElemFp8 ? rplane + (((uint64_t)rb * f.spr2 + cb * 8) * 3 * kLanes + L) * 4
                                             : rplane + ((uint64_t)slot0 * kLanes + L) * 16;
        float accA = 0.f, accB = 0.f;

        auto consume = [&](uint32_t sc, const uint32_t p[4], const uint32_t qq[4]) {
            const uint32_t kc = cb * kCols + sc * 32 + 8 * q;
            if (MODE == kDequant) {
                if (kc < f.K16) {
                    uint16_t *o = (uint16_t *)a.out + (uint64_t)row0 * f.K16 + kc;
                    if (row0 + r < f.M) *(uint4 *)(o + (uint64_t)r * f.K16) = make_uint4(p[0], p[1], p[2], p[3]);
                    if (row0 + r + 8 < f.M) *(uint4 *)(o + (uint64_t)(r + 8) * f.K16) = make_uint4(qq[0], qq[1], qq[2], qq[3]);
                }
            } else if (XBF16) {
                const uint4 xv = *(const uint4 *)((const uint16_t *)a.x + kc);
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    accA = dot2_bf16(p[k], u4_get(xv, k), accA);
                    accB = dot2_bf16(qq[k], u4_get(xv, k), accB);
                }
            } else {
                const float4 x0 = ((const float4 *)((const float *)a.x + kc))[0], x1 = ((const float4 *)((const float *)a.x + kc))[1];
                const float xf[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    accA = fmaf(bf16_lo(p[k]), xf[2 * k], accA); accA = fmaf(bf16_hi(p[k]), xf[2 * k + 1], accA);
                    accB = fmaf(bf16_lo(qq[k]), xf[2 * k], accB); accB = fmaf(bf16_hi(qq[k]), xf[2 * k + 1], accB);
                }
            }
        };

        if (ELEM == kElemFp8) {
            const uint32_t nsp = (nsc + 1) / 2;
            for (uint32_t sp = 0; sp < nsp; sp++) {
                const uint8_t *pp = rp + (uint64_t)sp * 3 * kLanes * 4;
                const uint32_t c0 = ldnt1(pp);
                const uint32_t c1 = ldnt1((pp + kLanes * 4));
                const uint32_t c2 = ldnt1((pp + 2 * kLanes * 4));
                uint32_t p[4], qq[4];
                const uint2 n0 = ldnt2((np + (uint64_t)(2 * sp) * kLanes * 8));
                decode_sc<ELEM, 0>(tab, &ms, n0, make_uint4(0, 0, 0, 0), c0, c1, c2, p, qq);
                consume(2 * sp, p, qq);
                if (2 * sp + 1 < nsc) {
                    const uint2 n1 = ldnt2((np + (uint64_t)(2 * sp + 1) * kLanes * 8));
                    decode_sc<ELEM, 4>(tab, &ms, n1, make_uint4(0, 0, 0, 0), c0, c1, c2, p, qq);
                    consume(2 * sp + 1, p, qq);
                }
            }
        } else {
            uint2 nn = ldnt2(np);
            uint4 rr = ldnt4(rp);
            for (uint32_t sc = 0; sc < nsc; sc++) {
                const uint2 nib = nn;
                const uint4 raw = rr;
                if (sc + 1 < nsc) {
                    nn = ldnt2((np + (uint64_t)(sc + 1) * kLanes * 8));
                    rr = ldnt4((rp + (uint64_t)(sc + 1) * kLanes * 16));
                }
                uint32_t p[4], qq[4];
                decode_sc<ELEM, 0>(tab, nullptr, nib, raw, 0u, 0u, 0u, p, qq);
                consume(sc, p, qq);
            }
        }

        // exceptions: planes decoded to +-0, the entries carry the value
        uint32_t cnt;
        const uint8_t *ep = exc_start(a, b, L, esz, cnt);
        float eA = 0.f, eB = 0.f;
        for (uint32_t k = 0; k < cnt; k++, ep += esz) {
            const uint32_t i = ep[0], j = i & 15;
            const uint32_t col = cb * kCols + (i >> 4) * 32 + frag_col(L, j), upper = (j >> 1) & 1u;
            const float w = exc_value<ELEM>(ep);
            if (MODE == kDequant) {
                ((uint16_t *)a.out)[(uint64_t)(row0 + r + 8 * upper) * f.K16 + col] = (uint16_t)f32_to_bf16_rne(w);
                continue;
            }
            const float xv = XBF16 ? __uint_as_float((uint32_t)((const uint16_t *)a.x)[col] << 16) : ((const float *)a.x)[col];
            if (upper) eB = fmaf(w, xv, eB); else eA = fmaf(w, xv, eA);
        }
        if (MODE != kDequant) {
            accA += eA; accB += eB;
            accA += xor_f<1>(accA); accA += xor_f<2>(accA);
            accB += xor_f<1>(accB); accB += xor_f<2>(accB);
            if (q == 0) {
                part[(g * kRows12 + r) * f.CB + cb] = accA;
                part[(g * kRows12 + r + 8) * f.CB + cb] = accB;
            }
        }
    }
    if (MODE != kDequant) finish_rows<MODE>(a, part, rg0 * kRows12, ng * kRows12, f.CB, ELEM == kElemFp8 ? &fin : nullptr);
}

// BF16 token path: a workgroup owns G whole 16-row groups; each half-wave decodes super-chunks sc0 .. sc0 + NS - 1
// of a block (SP = 16 / NS half-waves per block, so small matrices still fill the CUs; several blocks in turn when
// the tile has more than fit), with its
// nibble and raw loads four super-chunks ahead, the BF16 activations staged once per workgroup in LDS, and its lane's
// exceptions whose super-chunk lies in its range (the fp32 path keeps k_layout2 and its fp32 products).  Partial row sums per (row, column block, part), summed in a fixed
// order by the workgroup.  The fixed-width format needs no index to start inside a block.
template <int MODE, bool XBF16, int NS>
__global__ void __launch_bounds__(1024) k_layout2s(BlockArgs a) {
    static_assert(NS == 4 || NS == 8 || NS == 16, "four, two or one half-wave per block");
    static_assert(MODE == kToken && XBF16, "the BF16 token path");
    constexpr uint32_t SP = 16u / NS, R = 4;
    extern __shared__ uint32_t dyn[];
    const RankTab tab{a.lut[0], a.lut[1], a.lut[2], a.lut[3]};
    constexpr uint32_t esz = 3u;
    const uint32_t tid = threadIdx.x, nth = blockDim.x, L = tid & 31, r = L >> 2, q = L & 3;
    const uint32_t hw = tid >> 5, H = nth >> 5;
    const Shape f(a.M, a.K, 2);
    const uint32_t n8 = (f.K16 + 31u) / 32u * 4u;                   // x: K32 BF16 values, in chunks of eight
    uint4 *xs = (uint4 *)dyn;
    float *part = (float *)(xs + n8);
    const uint8_t *rplane = a.low + f.nib2_bytes();
    const uint32_t rg0 = blockIdx.x * a.G;
    const uint32_t ng = min(a.G, f.groups() - rg0);
    const uint32_t nt = ng * f.CB;
    for (uint32_t i = tid; i < n8; i += nth) xs[i] = ((const uint4 *)a.x)[i];
    __syncthreads();
    for (uint32_t it = hw; it < nt * SP; it += H) {
        const uint32_t t = it / SP, p = it - t * SP;
        const uint32_t g = t / f.CB, cb = t - g * f.CB, rb = rg0 + g, b = rb * f.CB + cb;
        const uint32_t nsc = ((cb == f.CB - 1 ? f.nl : 32u) + 1) / 2, slot0 = rb * f.spr + cb * 16;
        const uint32_t sc0 = p * NS, ns = sc0 < nsc ? min(NS, nsc - sc0) : 0u;
        const uint8_t *np = a.low + ((uint64_t)(slot0 + sc0) * kLanes + L) * 8;
        const uint8_t *rp = rplane + ((uint64_t)(slot0 + sc0) * kLanes + L) * 16;
        // the ring: super-chunk i of the range in slot i % R; loads past the range re-read its last super-chunk
        uint2 nr[R];
        uint4 rr[R];
        const uint32_t last = ns ? ns - 1u : 0u;
#pragma unroll
        for (uint32_t i = 0; i < R; i++) {
            nr[i] = ldnt2(np + (uint64_t)min(i, last) * kLanes * 8);
            rr[i] = ldnt4(rp + (uint64_t)min(i, last) * kLanes * 16);
        }
        float accA = 0.f, accB = 0.f;
#pragma unroll
        for (uint32_t i = 0; i < NS; i++) {
            if (i >= ns) continue;                               // a last column block's missing super-chunks
            uint32_t pa[4], qa[4];
            decode_sc<kElemBf16, 0>(tab, nullptr, nr[i % R], rr[i % R], 0u, 0u, 0u, pa, qa);
            if (i + R < NS) {
                nr[i % R] = ldnt2(np + (uint64_t)min(i + R, last) * kLanes * 8);
                rr[i % R] = ldnt4(rp + (uint64_t)min(i + R, last) * kLanes * 16);
            }
            const uint4 xv = xs[(cb * kCols + (sc0 + i) * 32u + 8u * q) >> 3];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                accA = dot2_bf16(pa[k], u4_get(xv, k), accA);
                accB = dot2_bf16(qa[k], u4_get(xv, k), accB);
            }
            asm volatile("" : "+v"(accA), "+v"(accB));
        }
        // exceptions of this lane whose super-chunk is in the range (planes decoded to +-0, the entries carry the value)
        uint32_t cnt;
        const uint8_t *ep = exc_start(a, b, L, esz, cnt);
        for (uint32_t k = 0; k < cnt; k++, ep += esz) {
            const uint32_t i = ep[0], j = i & 15, sc = i >> 4;
            if (sc - sc0 >= ns) continue;
            const uint32_t col = cb * kCols + sc * 32 + frag_col(L, j), upper = (j >> 1) & 1u;
            const float w = exc_value<kElemBf16>(ep);
            const float xv = __uint_as_float((uint32_t)((const uint16_t *)xs)[col] << 16);
            if (upper) accB = fmaf(w, xv, accB);
            else accA = fmaf(w, xv, accA);
        }
        accA += xor_f<1>(accA); accA += xor_f<2>(accA);
        accB += xor_f<1>(accB); accB += xor_f<2>(accB);
        if (q == 0) {
            const uint32_t pi = ((g * kRows12 + r) * f.CB + cb) * SP + p;
            part[pi] = accA;
            part[pi + 8u * f.CB * SP] = accB;
        }
    }
    finish_rows<MODE>(a, part, rg0 * kRows12, ng * kRows12, f.CB * SP);
}

// Row gather: one half-wave per requested row; the row's lanes store their columns, then patch their exceptions.
template <int ELEM>
__global__ void __launch_bounds__(256) k_gather2(GatherArgs a) {
    __shared__ MantLds ms;
    if (ELEM == kElemFp8) stage_mant(ms);
    const RankTab tab{a.lut[0], a.lut[1], a.lut[2], a.lut[3]};
    constexpr uint32_t esz = ELEM == kElemFp8 ? 2u : 3u;
    const uint32_t L = threadIdx.x & 31, r = L >> 2, q = L & 3;
    const Shape f(a.M, a.K, 2);
    // four half-waves per (id, column block), each a quarter of its super-chunks (4p .. 4p + 3): the fixed-width planes
    // need no cursor, so every super-chunk's loads go out together and a lookup waits one round trip, not sixteen
    const uint32_t item = blockIdx.x * (blockDim.x >> 5) + (threadIdx.x >> 5), pair = item >> 2, p = item & 3u;
    const uint32_t id = pair / f.CB, cb = pair - id * f.CB;
    if (id >= a.n_ids) return;
    const int64_t R = a.ids[id];
    if (R < 0 || R >= (int64_t)a.M) return;
    const uint32_t nsc = ((cb == f.CB - 1 ? f.nl : 32u) + 1) / 2, sc0 = 4u * p;
    if (sc0 >= nsc) return;
    const uint32_t last = min(4u, nsc - sc0) - 1u;            // super-chunks past the block's last re-read it
    const uint8_t *rplane = a.low + f.nib2_bytes();
    const uint32_t rb = (uint32_t)R / kRows12, rr = (uint32_t)R % kRows12;
    const bool mine = (rr & 7u) == r, upper = rr >= 8;
    uint16_t *o = a.out + (uint64_t)id * f.K16;
    const uint32_t slot0 = rb * f.spr + cb * 16;
    const uint8_t *np = a.low + ((uint64_t)(slot0 + sc0) * kLanes + L) * 8;
    uint2 nib[4];
    uint4 raw[4];
    uint32_t c[2][3];
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) nib[i] = *(const uint2 *)(np + (uint64_t)min(i, last) * kLanes * 8);
    if constexpr (ELEM == kElemFp8) {                          // 3-bit fields per pair of super-chunks (sc0 is even)
        const uint8_t *rp = rplane + (((uint64_t)rb * f.spr2 + cb * 8 + sc0 / 2u) * 3 * kLanes + L) * 4;
#pragma unroll
        for (uint32_t h = 0; h < 2; h++) {
            const uint8_t *pp = rp + (uint64_t)min(h, last / 2u) * 3 * kLanes * 4;
#pragma unroll
            for (uint32_t w = 0; w < 3; w++) c[h][w] = *(const uint32_t *)(pp + w * kLanes * 4);
        }
    } else {
        const uint8_t *rp = rplane + ((uint64_t)(slot0 + sc0) * kLanes + L) * 16;
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) raw[i] = *(const uint4 *)(rp + (uint64_t)min(i, last) * kLanes * 16);
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
        if (i > last) break;
        uint32_t pv[4], qv[4];
        if constexpr (ELEM == kElemFp8) {
            if (i & 1u) decode_sc<ELEM, 4>(tab, &ms, nib[i], make_uint4(0, 0, 0, 0), c[i / 2][0], c[i / 2][1], c[i / 2][2], pv, qv);
            else decode_sc<ELEM, 0>(tab, &ms, nib[i], make_uint4(0, 0, 0, 0), c[i / 2][0], c[i / 2][1], c[i / 2][2], pv, qv);
        } else {
            decode_sc<ELEM, 0>(tab, nullptr, nib[i], raw[i], 0u, 0u, 0u, pv, qv);
        }
        const uint32_t kc = cb * kCols + (sc0 + i) * 32 + 8 * q;
        if (mine && kc < f.K16) {
            const uint32_t *v = upper ? qv : pv;
            *(uint4 *)(o + kc) = make_uint4(v[0], v[1], v[2], v[3]);
        }
    }
    // exceptions of this lane in this quarter's super-chunks, after its plane values (the planes decode them to +-0);
    // the whole half computes the prefix over the lanes' counts, only the row's lanes use it
    const uint32_t b = rb * f.CB + cb;
    const uint32_t cnt = a.hdr[(uint64_t)b * kHdrBytes + L];
    const uint32_t incl = half_scan_incl(cnt, L);
    const uint8_t *ep = a.data + a.bases[b] + (uint64_t)(incl - cnt) * esz;
    if (mine) {
        for (uint32_t k = 0; k < cnt; k++, ep += esz) {
            const uint32_t i = ep[0], j = i & 15, sc = i >> 4;
            if (sc - sc0 > last || (((j >> 1) & 1u) != 0) != upper) continue;
            o[cb * kCols + sc * 32 + frag_col(L, j)] = (uint16_t)f32_to_bf16_rne(exc_value<ELEM>(ep));
        }
    }
}

template <int ELEM, int MODE, bool XBF16>
static int launch_fixed_t(const LaunchPlan &p, const BlockArgs &a, hipStream_t st) {
    if constexpr (ELEM == kElemBf16 && MODE == kToken && XBF16) {
        if (p.split) {
            if (p.split == 4) hipLaunchKernelGGL((k_layout2s<MODE, XBF16, 4>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
            else if (p.split == 2) hipLaunchKernelGGL((k_layout2s<MODE, XBF16, 8>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
            else hipLaunchKernelGGL((k_layout2s<MODE, XBF16, 16>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
            return (int)hipGetLastError();
        }
    }
    hipLaunchKernelGGL((k_layout2<ELEM, MODE, XBF16>), dim3(p.grid), dim3(p.threads), p.lds, st, a);
    return (int)hipGetLastError();
}

int launch_fixed(const LaunchPlan &p, int elem_t, int mode, bool xbf16, const BlockArgs &a, hipStream_t st) {
    if (elem_t == kElemFp8) {
        if (mode == kDequant) return launch_fixed_t<kElemFp8, kDequant, true>(p, a, st);
        if (mode == kF32) return launch_fixed_t<kElemFp8, kF32, false>(p, a, st);
        return xbf16 ? launch_fixed_t<kElemFp8, kToken, true>(p, a, st) : launch_fixed_t<kElemFp8, kToken, false>(p, a, st);
    }
    if (mode == kDequant) return launch_fixed_t<kElemBf16, kDequant, true>(p, a, st);
    if (mode == kF32) return launch_fixed_t<kElemBf16, kF32, false>(p, a, st);
    return xbf16 ? launch_fixed_t<kElemBf16, kToken, true>(p, a, st) : launch_fixed_t<kElemBf16, kToken, false>(p, a, st);
}

int launch_gather_fixed(int elem_t, const GatherArgs &a, hipStream_t st) {
    const uint32_t per = 8;                                        // half-wave items per workgroup
    const uint64_t items = (uint64_t)a.n_ids * Shape(a.M, a.K, 2).CB * 4u;
    const dim3 grid((uint32_t)((items + per - 1) / per));
    if (elem_t == kElemFp8) hipLaunchKernelGGL(k_gather2<kElemFp8>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(k_gather2<kElemBf16>, grid, dim3(256), 0, st, a);
    return (int)hipGetLastError();
}

}  // namespace nwc
