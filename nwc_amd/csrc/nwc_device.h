// nwc_device.h -- gfx950 building blocks shared by the kernels: the prefix-code window decoder, the staged decode
// table, half-wave scans/reductions and BF16 helpers.
//
// Execution model: a wave64 carries two independent blocks, one per 32-lane half, because the format fixes 32 lane
// streams per block (docs/format.md section 3).  All cross-lane traffic stays inside a half.
#pragma once
#include "nwc_format.h"

namespace nwc {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}
__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }
// round to nearest even (NaN stays NaN)
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// streaming (non-temporal) loads of plane data that is read exactly once
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;
__device__ __forceinline__ uint4 ldnt4(const void *p) {
    const u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldnt2(const void *p) {
    const u32x2_t v = __builtin_nontemporal_load((const u32x2_t *)p);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ldnt1(const void *p) { return __builtin_nontemporal_load((const uint32_t *)p); }

// Byte selectors for v_perm_b32(e, raw, sel): bytes 0-3 of `raw`, 4-7 of `e` (e byte 1/2 = exponent bytes of the
// pair), 0x0C = zero byte.  A BF16 pair [raw_j | e1][raw_j+1 | e2] (j = 0 or 2 inside the raw word):
constexpr uint32_t kSelPair0 = 0x06010500u;   // weights 0,1 of a raw word
constexpr uint32_t kSelPair2 = 0x06030502u;   // weights 2,3
// fp32 weights [0][0][raw_j][e_b] for the fp32-activation path
__device__ __forceinline__ constexpr uint32_t sel_f32(uint32_t j, uint32_t eb) { return (eb << 24) | (j << 16) | 0x0C0Cu; }

// ---- half-wave (32-lane) cross-lane operations ----
// Inclusive prefix sum inside each 32-lane half: DPP row shifts within 16-lane rows, then row 1 (3) adds the last
// lane of row 0 (2).
__device__ __forceinline__ uint32_t half_scan_incl(uint32_t v, uint32_t L) {
    (void)L;
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);   // row_shr:1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);   // row_shr:2
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);   // row_shr:4
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);   // row_shr:8
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);   // row_bcast:15 into rows 1, 3
    return v;
}
// value of lane `m ^ L` inside the 32-lane half (ds_swizzle bit mode: and 0x1F, or 0, xor m)
template <int M>
__device__ __forceinline__ float xor_f(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (M << 10) | 0x1F));
}

// Transposed reduction of 8 row sums over the 32 lanes of a half: afterwards lane L with (L & 3) == 0 holds the sum
// of row L >> 2 (9 exchanges instead of 8 x 5).
__device__ __forceinline__ float reduce8_transposed(float acc[8], uint32_t L) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const bool up = L & 16;
        float send = up ? acc[i] : acc[i + 4], keep = up ? acc[i + 4] : acc[i];
        acc[i] = keep + xor_f<16>(send);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const bool up = L & 8;
        float send = up ? acc[i] : acc[i + 2], keep = up ? acc[i + 2] : acc[i];
        acc[i] = keep + xor_f<8>(send);
    }
    const bool up = L & 4;
    float send = up ? acc[0] : acc[1], keep = up ? acc[1] : acc[0];
    float v = keep + xor_f<4>(send);
    v += xor_f<2>(v);
    v += xor_f<1>(v);
    return v;
}

// The same for 4 row sums: afterwards lane L with (L & 7) == 0 holds the sum of row L >> 3.
__device__ __forceinline__ float reduce4_transposed(float acc[4], uint32_t L) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const bool up = L & 16;
        float send = up ? acc[i] : acc[i + 2], keep = up ? acc[i + 2] : acc[i];
        acc[i] = keep + xor_f<16>(send);
    }
    const bool up = L & 8;
    float send = up ? acc[0] : acc[1], keep = up ? acc[1] : acc[0];
    float v = keep + xor_f<8>(send);
    v += xor_f<4>(v);
    v += xor_f<2>(v);
    v += xor_f<1>(v);
    return v;
}

// The same for 2 row sums: afterwards lane L with (L & 15) == 0 holds the sum of row L >> 4.
__device__ __forceinline__ float reduce2_transposed(float acc[2], uint32_t L) {
    const bool up = L & 16;
    float send = up ? acc[0] : acc[1], keep = up ? acc[1] : acc[0];
    float v = keep + xor_f<16>(send);
    v += xor_f<8>(v);
    v += xor_f<4>(v);
    v += xor_f<2>(v);
    v += xor_f<1>(v);
    return v;
}

// ---- decode table in LDS ----
// The stored 4096-word LUT is re-encoded once per workgroup.  For entries that are two complete codes byte 0 (c = bits
// of both codes, 4..12) becomes
//   kLutWindow: 32 - c, the funnel shift that advances a register window by c (Window);
//   kLutSeq:    17 - c, the right shift that puts the second code pair's 12 bits at [13:2] of the Seq cursor's
//               window (which starts one bit early); two entries added give 34 - (c1 + c2) in byte 0.
// Bytes 1/2 keep the two exponent bytes and byte 3 is 0.  The other entries (slow path) become: kLutWindow, the stored
// entry with bit 31; kLutSeq, exactly kSeqSlow, so that a step's sum (Seq::fast_quad) is at least kSeqSlowTest when
// either entry is slow and below it when both are fast (their bytes sum to less than 2^26).
enum LutKind { kLutWindow = 0, kLutSeq = 1 };
constexpr uint32_t kSeqSlow = 0x40000000u, kSeqSlowTest = 0x20000000u;

template <int PEEK> struct LutT {
    uint32_t tab[1u << PEEK];
    alignas(16) uint8_t eor[16];    // exp_of_rank, read back from the table (the slow path's rank -> byte map)
};
using LutLds = LutT<kPeek>;
using LutLds13 = LutT<kPeekSeq>;

template <int KIND>
__device__ __forceinline__ uint32_t lut_transform(uint32_t e) {
    if (e & kFlag) return KIND == kLutWindow ? e | 0x80000000u : kSeqSlow;
    const uint32_t c = e & 0xFFu;
    return (e & 0xFFFFFF00u) | (KIND == kLutWindow ? ((32u - c) & 31u) : (29u - kPeek - c));
}

// Table staging in three parts so its loads overlap other requests: lut_issue reads the first 4 * blockDim 16-byte
// chunks (all 1024 for >= 256 threads) and the word exp_of_rank[tid & 15] comes from; lut_commit re-encodes and
// stores them; lut_finish copies any remaining chunks (fewer than 256 threads).  A kernel calls lut_finish only after
// every request that must not wait for the streams: the loads of its loop make the compiler wait for every
// outstanding load where the loop ends, even when it runs no iteration.  The caller publishes the table with a
// barrier.
struct LutLoad {
    u32x4_t v0, v1, v2, v3;
    uint32_t ew;
};
__device__ __forceinline__ void lut_issue(LutLoad &Q, const uint32_t *__restrict__ lut, uint32_t nth = blockDim.x) {
    const uint32_t tid = threadIdx.x;
    constexpr uint32_t n4 = kLutWords / 4;
    // source word of exp_of_rank[q]: pattern "q zeros, one, sign 0" for q < 11; ranks 11-14 sit in bytes 1/2 of
    // entries 0 and 1 (11, 13: byte 1; 12, 14: byte 2); slot 15 is unused
    const uint32_t q = tid & 15u;
    Q.ew = lut[q < 11u ? (1u << (kPeek - 1u - q)) : q < 15u ? (q - 11u) >> 1 : 0u];
    const u32x4_t *l4 = (const u32x4_t *)lut;
    Q.v0 = l4[min(tid, n4 - 1u)];
    Q.v1 = l4[min(tid + nth, n4 - 1u)];
    Q.v2 = l4[min(tid + 2u * nth, n4 - 1u)];
    Q.v3 = l4[min(tid + 3u * nth, n4 - 1u)];
}
template <int KIND>
__device__ __forceinline__ void lut_store4(LutLds &s, uint32_t i, u32x4_t e) {
#pragma unroll
    for (int j = 0; j < 4; j++) e[j] = lut_transform<KIND>(e[j]);
    ((u32x4_t *)s.tab)[i] = e;
}
template <int KIND>
__device__ __forceinline__ void lut_commit(LutLds &s, const LutLoad &Q, uint32_t nth = blockDim.x) {
    const uint32_t tid = threadIdx.x;
    constexpr uint32_t n4 = kLutWords / 4;
    if (tid < n4) lut_store4<KIND>(s, tid, Q.v0);
    if (tid + nth < n4) lut_store4<KIND>(s, tid + nth, Q.v1);
    if (tid + 2u * nth < n4) lut_store4<KIND>(s, tid + 2u * nth, Q.v2);
    if (tid + 3u * nth < n4) lut_store4<KIND>(s, tid + 3u * nth, Q.v3);
    const uint32_t q = tid & 15u;
    if (tid < 16) s.eor[tid] = q == 15u ? 0 : (uint8_t)((Q.ew >> ((q < 11u || (q & 1u)) ? 8u : 16u)) & 0x7Fu);
}
template <int KIND>
__device__ __forceinline__ void lut_finish(LutLds &s, const uint32_t *__restrict__ lut, uint32_t nth = blockDim.x) {
    const uint32_t tid = threadIdx.x;
    constexpr uint32_t n4 = kLutWords / 4;
    for (uint32_t i = tid + 4u * nth; i < n4; i += nth) lut_store4<KIND>(s, i, ((const u32x4_t *)lut)[i]);   // < 256 threads
}
template <int KIND>
__device__ __forceinline__ void stage_lut(LutLds &s, const uint32_t *__restrict__ lut) {
    LutLoad Q;
    lut_issue(Q, lut);
    lut_commit<KIND>(s, Q);
    lut_finish<KIND>(s, lut);
    __syncthreads();
}

template <int PEEK>
__device__ __forceinline__ uint32_t lds_entry(const LutT<PEEK> &s, uint32_t byte_off) {
    return *(const uint32_t *)((const char *)s.tab + byte_off);
}

// The 13-bit table (nwc_seq_table: entries already encoded, exp_of_rank in the last four words) copied into LDS:
// three 16-byte chunks per thread for >= 683 threads, then the rest; the caller publishes it with a barrier.
struct SeqLoad {
    u32x4_t v0, v1, v2;
};
__device__ __forceinline__ void seq_issue(SeqLoad &Q, const uint32_t *__restrict__ tab, uint32_t nth = blockDim.x) {
    const uint32_t tid = threadIdx.x;
    constexpr uint32_t n4 = kSeqTableWords / 4;
    const u32x4_t *t4 = (const u32x4_t *)tab;
    Q.v0 = t4[min(tid, n4 - 1u)];
    Q.v1 = t4[min(tid + nth, n4 - 1u)];
    Q.v2 = t4[min(tid + 2u * nth, n4 - 1u)];
}
__device__ __forceinline__ void seq_store(LutLds13 &s, uint32_t i, u32x4_t v) {
    constexpr uint32_t n4 = kSeqTableWords / 4;
    if (i < n4 - 1u) ((u32x4_t *)s.tab)[i] = v;
    else if (i == n4 - 1u) *(u32x4_t *)s.eor = v;                      // the last chunk: exp_of_rank
}
__device__ __forceinline__ void seq_commit(LutLds13 &s, const SeqLoad &Q, uint32_t nth = blockDim.x) {
    const uint32_t tid = threadIdx.x;
    seq_store(s, tid, Q.v0);
    seq_store(s, tid + nth, Q.v1);
    seq_store(s, tid + 2u * nth, Q.v2);
}
// the chunks past the first three per thread (fewer than 683 threads); called as lut_finish is
__device__ __forceinline__ void seq_finish(LutLds13 &s, const uint32_t *__restrict__ tab, uint32_t nth = blockDim.x) {
    const uint32_t tid = threadIdx.x;
    constexpr uint32_t n4 = kSeqTableWords / 4;
    for (uint32_t i = tid + 3u * nth; i < n4; i += nth) seq_store(s, i, ((const u32x4_t *)tab)[i]);
}

// ---- prefix-code window ----
// hi:lo is a 64-bit MSB-first window holding `avail` valid bits (>= 32 between steps); w is the next stream word and
// wn the one after it, both already read; p points at wn.  Bits below the valid ones are zero.  P is the word
// pointer type: an LDS slot (the block's streams staged once) or global memory (fallback).  The fast path reads
// wn for the next step unconditionally, so no step waits for its own refill read.
template <int ELEM, typename P>
struct Window {
    P p;
    uint32_t hi, lo, w, wn, avail;

    __device__ __forceinline__ void init(P lane_words) {
        hi = lane_words[0]; lo = lane_words[1]; w = lane_words[2]; wn = lane_words[3];
        p = lane_words + 3;
        avail = 64;
    }

    // advance by 1 <= c <= 24 bits and refill (slow path)
    __device__ __forceinline__ void consume(uint32_t c) {
        hi = __builtin_amdgcn_alignbit(hi, lo, 32u - c);
        lo <<= c;
        avail -= c;
        if (avail < 32) {
            hi |= w >> avail;
            lo |= w << (32u - avail);
            avail += 32;
            w = wn;
            wn = *++p;
        }
    }

    // one code by counting leading zeros: rank r < max -> r zeros, one, sign; BF16 escape -> 15 zeros, one, byte
    __device__ __forceinline__ uint32_t one_code(const LutLds &s) {
        uint32_t u = __clz((int)hi);
        if (ELEM == kElemFp8 || u < kMaxRankBf16) {
            u = u < 15u ? u : 15u;
            const uint32_t b = (((hi >> (30u - u)) & 1u) << 7) | s.eor[u];
            consume(u + 2);
            return b;
        }
        consume(16);
        const uint32_t b = hi >> 24;
        consume(8);
        return b;
    }

    // Four codes = two pairs.  Returns e1 with the exponent bytes of weights 0,1 in bytes 1,2 and e2 with those of
    // weights 2,3.  Fast path: two table reads (the second at the window shifted by the first pair), one window
    // advance for both pairs, at most one refill.
    __device__ __forceinline__ void quad(const LutLds &s, uint32_t &e1, uint32_t &e2) {
        e1 = lds_entry(s, (hi >> 18) & 0x3FFCu);
        const uint32_t t = __builtin_amdgcn_alignbit(hi, 0u, e1);      // hi << c1
        e2 = lds_entry(s, (t >> 18) & 0x3FFCu);
        if ((int)(e1 | e2) < 0) {
            uint32_t bytes = 0;                                        // b3 b2 b1 b0 after four codes
#pragma unroll 1
            for (int k = 0; k < 4; k++) bytes = (bytes >> 8) | (one_code(s) << 24);
            e1 = (bytes << 8) & 0x00FFFF00u;
            e2 = (bytes >> 8) & 0x00FFFF00u;
        } else {
            const uint32_t d = e1 + e2;                                // low 5 bits: 32 - (c1 + c2) mod 32
            uint32_t nhi = __builtin_amdgcn_alignbit(hi, lo, d);
            uint32_t nlo = __builtin_amdgcn_alignbit(lo, 0u, d);
            const uint32_t tt = avail + (d & 0xFFu);                  // avail - c1 - c2 + 64, in [72, 128)
            const bool need = tt < 96;                                 // fewer than 32 valid bits left
            const uint32_t ins = need ? w : 0u;
            nhi |= __builtin_amdgcn_alignbit(0u, ins, tt);             // ins >> avail'
            nlo |= __builtin_amdgcn_alignbit(ins, 0u, tt);             // ins << (32 - avail')
            hi = nhi; lo = nlo;
            avail = (tt & ~0x60u) | 0x20u;                             // avail' (+32 if refilled)
            w = need ? wn : w;
            p += need ? 1 : 0;
            wn = *p;                                                   // used from the next step on
        }
    }

    // skip four codes (gather: rows in front of the wanted one)
    __device__ __forceinline__ void skip_quad(const LutLds &s) { uint32_t a, b; quad(s, a, b); }
};

// ---- bit cursor over an LDS-staged lane stream ----
// P = bit position of the next code (0 = the MSB of the lane's word 0).  The cursor works one bit behind it, at Q = P - 1:
// it keeps the word pointer wp = lane + ((Q - 1) >> 5), the words A = wp[0], B = wp[1], C = wp[2], and a shift s with
// s & 31 = 31 - ((Q - 1) & 31), so that the 32 bits from Q are alignbit(A, B, s): a don't-care bit (already consumed)
// on top of the next 31.  s holds (s & 31) - 32 (bits 5-31 set; -32 is an inline constant of the instruction that
// forms it).  Both choices serve one add: with table entries whose byte 0 is 29 - PEEK - c (16 - c for the 13-bit
// table), e1 + e2 + s is (s & 31) - (c1 + c2) plus the exponent bytes' sums above byte 0, with no constant to add (a
// cursor at P would need one).  An advance by c <= 24 bits moves at most one word, exactly
// when that value is negative (bit 7): A, B <- B, C, and the new C is read for the step after next, so no read of
// stream words lies on the dependency chain of a step:
//   window -> table read (kLutSeq encoding) -> shift -> table read -> add -> test -> select -> window.
// The words may live in LDS (staged streams) or global memory (fallback).  STRIDE is the distance in words between
// consecutive words of a lane (1 for a lane stream stored contiguously; kLanes for 32 lanes interleaved word by word).
template <int ELEM, int STRIDE = 1>
struct Seq {
    const uint32_t *wp;
    uint32_t s;
    uint32_t A, B, C;

    // P = 0: Q - 1 = -2 lies in word -1 and s & 31 = 1, so A supplies only the window's don't-care top bit: it is set
    // to 0 and word -1 is never read (in global memory it may precede the allocation).
    __device__ __forceinline__ void init(const uint32_t *lane) {
        wp = lane - STRIDE;
        s = 1u | 0xFFFFFFE0u;
        A = 0u; B = lane[0]; C = lane[STRIDE];
    }
    // start at bit position P of the lane's stream (any P >= 0)
    __device__ __forceinline__ void init_at(const uint32_t *lane, uint32_t P) {
        const int32_t m = (int32_t)P - 2;
        wp = lane + (m >> 5) * STRIDE;
        s = (31u - ((uint32_t)m & 31u)) | 0xFFFFFFE0u;
        reload();
    }
    // the bit position of the next code
    __device__ __forceinline__ uint32_t position(const uint32_t *lane) const {
        return (uint32_t)((wp - lane) / STRIDE) * 32u + 33u - (s & 31u);
    }
    __device__ __forceinline__ uint32_t window() const { return __builtin_amdgcn_alignbit(A, B, s); }
    // t = (s & 31) - c as an 8-bit two's complement value in its low byte (higher bits are don't-care); bit 7 says the
    // cursor crossed into the next word
    __device__ __forceinline__ void step(uint32_t t) {
        const uint32_t x = __builtin_amdgcn_ubfe(t, 7, 1);
        const bool crossed = x != 0u;
        s = (t & 31u) | 0xFFFFFFE0u;
        A = crossed ? B : A;
        B = crossed ? C : B;
        wp += x * STRIDE;
        C = wp[2 * STRIDE];
    }
    // re-read the cached words after the position was reset.  A is dead when s & 31 = 0 and gives only the don't-care
    // bit when s & 31 = 1, so it is read from wp[STRIDE] then (at P = 0, wp[0] is word -1)
    __device__ __forceinline__ void reload() { A = wp[(s & 31u) <= 1u ? STRIDE : 0]; B = wp[STRIDE]; C = wp[2 * STRIDE]; }

    // Four codes = two pairs from two table reads; e1 holds the exponent bytes of weights 0,1 in bytes 1,2 and e2
    // those of weights 2,3.  With a PEEK-bit table (13: nwc_seq_table; 12: the stored LUT re-encoded) byte 0 of an
    // entry is 29 - PEEK - c, so e1 + e2 + s is (s & 31) - c + 2 (13 - PEEK) plus the exponent bytes' sums from byte 1
    // on: the 13-bit table needs no constant, and the low byte is (s & 31) - c.  Returns t: the step is correct only
    // if t < kSeqSlowTest (either entry slow: at least 2^30; both fast: below 2^26, except when all four exponent
    // bytes are 0 and the low byte borrows, which reads as slow and is merely redone); otherwise the caller resets the
    // position and redoes the step with slow_quad.
    template <int PEEK>
    __device__ __forceinline__ uint32_t fast_quad(const LutT<PEEK> &T, uint32_t &e1, uint32_t &e2) {
        constexpr uint32_t mask = ((1u << PEEK) - 1u) << 2;
        const uint32_t hi = window();
        e1 = lds_entry(T, (hi >> (29 - PEEK)) & mask);
        e2 = lds_entry(T, (hi >> (e1 & 31u)) & mask);                  // the PEEK bits after the first c1
        const uint32_t t = PEEK == 13 ? e1 + e2 + s : e1 + e2 + s - 2u * (13u - PEEK);
        step(t);
        return t;
    }

    // one code by counting leading zeros: rank r < max -> r zeros, one, sign; BF16 escape -> 15 zeros, one, byte
    template <int PEEK>
    __device__ __forceinline__ uint32_t slow_code(const LutT<PEEK> &T) {
        const uint32_t hi = window() << 1;                             // the bits from P (codes take at most 24)
        const uint32_t u = min((uint32_t)__clz((int)hi), 15u);
        const bool esc = ELEM != kElemFp8 && u >= kMaxRankBf16;       // BF16: 15 zeros, one, the byte
        const uint32_t br = (((hi >> (30u - u)) & 1u) << 7) | T.eor[u];
        const uint32_t b = esc ? (hi >> 8) & 0xFFu : br;             // no branch: the wave stays converged
        step((s & 31u) - (esc ? 24u : u + 2u));
        return b;
    }
    template <int PEEK>
    __device__ __forceinline__ void slow_quad(const LutT<PEEK> &T, uint32_t &e1, uint32_t &e2) {
        uint32_t bytes = 0;                                            // b3 b2 b1 b0 after four codes
#pragma unroll 1
        for (int k = 0; k < 4; k++) bytes = (bytes >> 8) | (slow_code(T) << 24);
        e1 = (bytes << 8) & 0x00FFFF00u;
        e2 = (bytes >> 8) & 0x00FFFF00u;
    }
};

// Per-block lane offsets: n = words of lane L, start = words of the lanes before it, total = words of the block.
struct LaneSpan { uint32_t n, start, total; };
__device__ __forceinline__ LaneSpan lane_span(const uint8_t *__restrict__ hdr, uint32_t b, uint32_t L) {
    LaneSpan r;
    r.n = hdr[(uint64_t)b * kHdrBytes + L];
    const uint32_t incl = half_scan_incl(r.n, L);
    r.start = incl - r.n;
    r.total = __shfl(incl, 31, 32);
    return r;
}

// Copies the 32 lane streams of a block (plus the window's read-ahead of two words) into the half-wave's LDS slot with
// 16-byte loads.  `sh` returns the word offset of the block inside the slot (bases[] are 8-byte aligned, the copy
// 16-byte aligned).  False when the block does not fit; the caller then decodes from global memory.
__device__ __forceinline__ bool stage_block(uint32_t *slot, uint32_t slot_words, const uint8_t *__restrict__ data,
                                            uint32_t base, uint32_t total, uint32_t L, uint32_t &sh) {
    const uint32_t a16 = base & ~15u;
    sh = (base & 15u) >> 2;
    const uint32_t need = sh + total + 3;
    if (need > slot_words) return false;
    for (uint32_t i = L * 4; i < need; i += 128) *(uint4 *)(slot + i) = *(const uint4 *)(data + a16 + 4u * i);
    __builtin_amdgcn_wave_barrier();
    return true;
}

// raw bytes of a lane's 16 weights for the PRMT stage: word k holds weights 4k..4k+3 (fp8: nibble << 4)
__device__ __forceinline__ uint4 expand_nibbles(uint2 c) {
    return make_uint4((c.x << 4) & 0xF0F0F0F0u, c.x & 0xF0F0F0F0u, (c.y << 4) & 0xF0F0F0F0u, c.y & 0xF0F0F0F0u);
}
__device__ __forceinline__ uint32_t u4_get(const uint4 &v, int k) { return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w; }

// Launch arguments shared by the block kernels.
struct BlockArgs {
    const uint8_t *data;
    const uint32_t *bases;
    const uint8_t *hdr;
    const uint32_t *lut;
    const uint8_t *low;
    const void *x;          // fp32 or BF16 activations
    const uint16_t *bias;   // BF16 [M] or null
    const float *scale;     // fp32 [M] or null
    void *out;              // token: BF16 y [M]; fp32 path: y [M]; dequant: BF16 [M x K16]; row index: u16 [nb x 3 x 32]
    const uint16_t *aux;    // layout 0 row index (bit positions of rows 2, 4, 6 per lane and block) or null
    uint32_t M, K;
    uint32_t G;             // row groups per workgroup
    uint32_t slot_words;    // LDS words per half-wave for a staged block (layouts 0/1)
    const uint32_t *seq;    // 13-bit token-path decode table (nwc_seq_table) or null
    uint32_t stride;        // layout 0 in fixed slots: block b's streams at byte b * stride (elem_stride); 0 = bases[b]
};

// Byte offset of block b's streams: computed for fixed slots, else bases[b] (a scalar load the stream copy waits for).
__device__ __forceinline__ uint32_t block_base(const BlockArgs &a, uint32_t b) {
    return a.stride ? b * a.stride : a.bases[b];
}

// Prefill without a temporary BF16 matrix (k_prefill0): the matrix in `a` (a.out = y [T x M] BF16, a.aux = row index,
// a.seq = 13-bit table, both required), activations [T x K16] BF16.
struct PrefillArgs {
    BlockArgs a;
    const uint16_t *xt;
    uint32_t T;
};

struct GatherArgs {
    const uint8_t *data;
    const uint32_t *bases;
    const uint8_t *hdr;
    const uint32_t *lut;
    const uint8_t *low;
    const int64_t *ids;
    uint32_t n_ids;
    uint16_t *out;
    uint32_t M, K;
    uint32_t slot_words;
};

enum Mode { kToken = 0, kDequant = 1, kF32 = 2, kRowIndex = 3 };

// Layout-0 row index: for block b, lane L and j = 0..2, the bit position (from the lane's first word) where row
// 2 (j + 1) of the lane's stream begins, at aux[(b * 3 + j) * 32 + L].  Built once per matrix (MODE kRowIndex); it lets
// several half-waves decode one block's rows in parallel.
constexpr uint32_t kRowIndexSplits = 3;

// The scale and bias of the first row a thread finishes (row0 + threadIdx.x), requested before the kernel's other
// loads so that the finish does not wait a memory round trip for them (and so that no later wait covers them).
// PRE = false loads nothing (kernels that keep the finish's own loads where a matrix rarely has either: the held
// registers and the branch cost more there than the round trip).
// The bias stays in its BF16 bits until the finish (widening it here would make the wave wait for the load).  `flags`
// (bit 0: scale, bit 1: bias) says which pointers are set when a kernel knows it without reading them: kFinishAll
// tests the pointers themselves.
struct RowFinish {
    float scale;
    uint32_t bias_bits;
};
constexpr uint32_t kFinishAll = 0xFFFFFFFFu;
template <int MODE, bool PRE = true>
__device__ __forceinline__ RowFinish row_finish_load(const BlockArgs &a, uint32_t row0, uint32_t nrows,
                                                     uint32_t flags = kFinishAll) {
    RowFinish r{1.f, 0u};
    const uint32_t row = row0 + threadIdx.x;
    if (PRE && MODE == kToken && threadIdx.x < nrows && row < a.M) {
        if (flags != kFinishAll) {
            if (flags & 1u) r.scale = a.scale[row];
            if (flags & 2u) r.bias_bits = a.bias[row];
        } else {
            if (a.scale) r.scale = a.scale[row];
            if (a.bias) r.bias_bits = a.bias[row];
        }
    }
    return r;
}

// Workgroup epilogue of the token / fp32 paths: rows of the tile summed over the column blocks (ascending),
// times scale, plus bias, rounded to BF16 (token) or written as fp32.  `pre`: this thread's first row's scale and
// bias, already loaded.
template <int MODE>
__device__ __forceinline__ void finish_rows(const BlockArgs &a, const float *part, uint32_t row0, uint32_t nrows, uint32_t CB,
                                            const RowFinish *pre = nullptr, uint32_t nth = blockDim.x) {
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < nrows; i += nth) {
        const uint32_t row = row0 + i;
        if (row >= a.M) break;
        float v = 0.f;
        for (uint32_t cb = 0; cb < CB; cb++) v += part[i * CB + cb];
        if (MODE == kToken) {
            const bool first = pre && i == threadIdx.x;
            if (a.scale) v *= first ? pre->scale : a.scale[row];
            if (a.bias) v += __uint_as_float((first ? pre->bias_bits : (uint32_t)a.bias[row]) << 16);
            ((uint16_t *)a.out)[row] = (uint16_t)f32_to_bf16_rne(v);
        } else {
            ((float *)a.out)[row] = v;
        }
    }
}

}  // namespace nwc
