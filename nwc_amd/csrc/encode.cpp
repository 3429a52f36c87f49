// encode.cpp -- host side of the C ABI: nwc_info, nwc_layout, nwc_encode, nwc_build_tab.
//
// The encoder produces the on-disk format v9/v10/v11 byte for byte (parda21/NWC csrc/nwc_ops.cu:175-348,
// docs/format.md sections 2-4d).  It is organised for a many-core host rather than as the reference's single
// loop: a parallel histogram, a parallel pass that sizes every lane stream / exception list, a serial prefix sum
// over blocks (which also reproduces the reference's failure codes in its serial order), and a parallel pass that
// writes every block straight to its final offset.  No temporary copy of the matrix is made.
#include "nwc_format.h"
#include "nwc_ops.h"

#include <algorithm>
#include <array>
#include <atomic>
#include <cmath>
#include <cstring>
#include <functional>
#include <sched.h>
#include <thread>
#include <vector>

using namespace nwc;

namespace {

int host_threads() {
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof set, &set) == 0) {
        int c = CPU_COUNT(&set);
        if (c > 0) return std::min(c, 64);
    }
    unsigned h = std::thread::hardware_concurrency();
    return h ? (int)std::min(h, 64u) : 1;
}

// Run f(begin, end) over [0, n) on up to host_threads() threads (inline when the range is small).
void parallel_range(uint64_t n, uint64_t min_chunk, const std::function<void(uint64_t, uint64_t)> &f) {
    int nt = host_threads();
    uint64_t chunks = std::max<uint64_t>(1, std::min<uint64_t>(nt, (n + min_chunk - 1) / std::max<uint64_t>(min_chunk, 1)));
    if (chunks <= 1) { if (n) f(0, n); return; }
    std::vector<std::thread> th;
    uint64_t per = (n + chunks - 1) / chunks;
    for (uint64_t c = 0; c < chunks; c++) {
        uint64_t a = c * per, b = std::min(n, a + per);
        if (a >= b) break;
        th.emplace_back(f, a, b);
    }
    for (auto &t : th) t.join();
}

// ---- fp8 e4m3fn byte -> (symbol, low bits) ----------------------------------------------------------------
// Derived from the fp32 bit pattern of the value: the decoder rebuilds fp32 [s | B3 | L | 0] where B3 is the fp32
// exponent >> 1 (the coded symbol's table byte) and L = (exponent & 1) << 7 | top mantissa bits.  Every finite
// e4m3 value has at most 3 significant mantissa bits after normalisation, so L carries it exactly.
struct Fp8Split {
    int8_t sym01[256];    // layouts 0/1: 10 symbols, -1 = NaN
    uint8_t nib01[256];   // layouts 0/1: 4-bit raw nibble (exponent low bit, 3 mantissa bits)
    int8_t sym2[256];     // layout 2: 20 symbols, -1 = NaN
    uint8_t m3_2[256];    // layout 2: 3-bit raw field
    uint8_t hb2[20];      // layout 2: table byte of a symbol
    uint8_t lb2[20];      // layout 2: low-byte bit 7 of a symbol
    Fp8Split() {
        memset(hb2, 0, sizeof hb2);
        memset(lb2, 0, sizeof lb2);
        for (int b = 0; b < 256; b++) {
            const uint32_t e = (b >> 3) & 15, m = b & 7;
            if (e == 15 && m == 7) { sym01[b] = sym2[b] = -1; nib01[b] = m3_2[b] = 0; continue; }
            float v = e ? std::ldexp(1.0f + m / 8.0f, (int)e - 7) : m * (1.0f / 512.0f);
            uint32_t u; memcpy(&u, &v, 4);
            const uint32_t ex = (u >> 23) & 0xFF, top3 = (u >> 20) & 7;
            const uint32_t b3 = ex >> 1;
            nib01[b] = (uint8_t)(((ex & 1) << 3) | top3);
            // layouts 0/1: symbols 0..7 are table bytes 60..67, 8 is byte 59, 9 is zero
            sym01[b] = (int8_t)(b3 >= 60 ? b3 - 60 : (b3 == 59 ? 8 : 9));
            // layout 2: symbols 1..15 are the normal exponents, 16..19 the subnormal groups m>=4, m=2|3, m=1, zero
            int s2 = e ? (int)e : (m >= 4 ? 16 : m >= 2 ? 17 : m == 1 ? 18 : 19);
            sym2[b] = (int8_t)s2;
            m3_2[b] = (uint8_t)top3;
            hb2[s2] = (uint8_t)b3;
            lb2[s2] = (uint8_t)((ex & 1) << 7);
        }
    }
};
const Fp8Split &fp8_tables() { static const Fp8Split t; return t; }

// ---- symbols ---------------------------------------------------------------------------------------------
// Per weight: `high` = sign << 7 | symbol, `low` = raw byte (BF16), nibble (fp8 layouts 0/1) or 3-bit field.
struct Splitter {
    const uint16_t *w16; const uint8_t *w8; bool fp8, l2;
    inline uint8_t high(uint64_t i) const {
        if (!fp8) return (uint8_t)(w16[i] >> 8);
        const uint8_t b = w8[i];
        const auto &T = fp8_tables();
        return (uint8_t)((b & 0x80) | (l2 ? T.sym2[b] : T.sym01[b]));
    }
    inline uint8_t low(uint64_t i) const {
        if (!fp8) return (uint8_t)w16[i];
        const auto &T = fp8_tables();
        return l2 ? T.m3_2[w8[i]] : T.nib01[w8[i]];
    }
};

// Symbol order by frequency.  The format fixes the tie-breaking: the reference ranks with an in-place exchange
// sort (nwc_ops.cu:193-194, :275-277) that is not stable, and exp_of_rank / the LUT record the result, so the
// same comparisons are made here.
void rank_symbols(const uint64_t hist[128], int nsym, int ord[128]) {
    for (int i = 0; i < 128; i++) ord[i] = i;
    for (int a = 0; a < nsym; a++)
        for (int b = a + 1; b < nsym; b++)
            if (hist[ord[b]] > hist[ord[a]]) std::swap(ord[a], ord[b]);
}

// MSB-first code words, little-endian 32-bit words in memory.
struct WordSink {
    uint8_t *dst; uint64_t acc = 0; int n = 0; uint32_t words = 0;
    inline void put(uint32_t v, int len) {
        acc = (acc << len) | v; n += len;
        if (n >= 32) { n -= 32; uint32_t w = (uint32_t)(acc >> n); memcpy(dst + 4ull * words++, &w, 4); }
    }
    inline void close() { if (n) { uint32_t w = (uint32_t)(acc << (32 - n)); memcpy(dst + 4ull * words++, &w, 4); n = 0; } }
};

inline uint64_t align8(uint64_t v) { return (v + 7) & ~7ull; }

// Stream position -> matrix element of a lane (layout 0 row-major lanes; layout 1 fragment order).
struct LanePos {
    uint32_t row, col;
};
inline LanePos lane_pos(int lay, uint32_t rb, uint32_t cb, uint32_t L, uint32_t i) {
    if (lay) return {rb * kRows12 + frag_row(L, i & 15), cb * kCols + (i >> 4) * 32 + frag_col(L, i & 15)};
    return {rb * kRows0 + (i >> 4), cb * kCols + L * 16 + (i & 15)};
}

// ---- layouts 0 and 1 -------------------------------------------------------------------------------------
int64_t encode_prefix(const Splitter &S, const Shape &f, uint64_t K, int t, int lay, uint16_t *psym, uint32_t *bases,
                      uint8_t *hdr, uint8_t *data, uint64_t cap, uint8_t *low) {
    const int nsym = t == kElemFp8 ? 10 : 128;
    const uint32_t maxr = t == kElemFp8 ? kMaxRankFp8 : kMaxRankBf16;
    const uint64_t n = (uint64_t)f.M * K;

    // histogram
    std::vector<std::array<uint64_t, 128>> part(host_threads() + 1);
    std::atomic<int> slot{0};
    parallel_range(n, 1u << 20, [&](uint64_t a, uint64_t b) {
        auto &h = part[slot++];
        h.fill(0);
        for (uint64_t i = a; i < b; i++) h[S.high(i) & 0x7F]++;
    });
    uint64_t hist[128] = {0};
    for (int s = 0; s < slot; s++) for (int k = 0; k < 128; k++) hist[k] += part[s][k];
    int ord[128];
    rank_symbols(hist, nsym, ord);
    uint8_t rank[128];
    for (int r = 0; r < 128; r++) rank[ord[r]] = (uint8_t)r;
    static const uint8_t kFp8Byte3[10] = {60, 61, 62, 63, 64, 65, 66, 67, 59, 0};
    for (uint32_t i = 0; i < kNpsym; i++) psym[i] = 0;
    for (int i = 0; i < 16; i++) psym[i] = (uint16_t)(t == kElemFp8 ? (i < 10 ? kFp8Byte3[ord[i]] : 0) : ord[i]);

    // code length of each high byte (sign | symbol)
    uint8_t clen[256];
    for (int h = 0; h < 256; h++) { uint32_t r = rank[h & 0x7F]; clen[h] = (uint8_t)(r < maxr ? r + 2 : 24); }

    // pass 1: words per lane
    std::vector<uint16_t> nwords((size_t)f.nb * kLanes);
    parallel_range(f.nb, 64, [&](uint64_t b0, uint64_t b1) {
        for (uint64_t b = b0; b < b1; b++) {
            const uint32_t rb = (uint32_t)(b / f.CB), cb = (uint32_t)(b % f.CB);
            const uint32_t nchunk = cb == f.CB - 1 ? f.nl : 32;
            const uint32_t npos = lay ? ((nchunk + 1) / 2) * 16 : kRows0 * 16;
            for (uint32_t L = 0; L < kLanes; L++) {
                uint64_t bits = 0;
                for (uint32_t i = 0; i < npos; i++) {
                    LanePos p = lane_pos(lay, rb, cb, L, i);
                    bits += (p.row >= f.M || p.col >= f.K) ? 2 : clen[S.high((uint64_t)p.row * K + p.col)];
                }
                uint64_t w = (bits + 31) / 32;
                nwords[b * kLanes + L] = (uint16_t)std::min<uint64_t>(w, 65535);
            }
        }
    });

    // serial prefix: block offsets; the reference fails with -1 at the first lane of more than 255 words or
    // whose end + 64 passes the capacity (nwc_ops.cu:311)
    uint64_t pos = 0;
    for (uint32_t b = 0; b < f.nb; b++) {
        pos = align8(pos);
        bases[b] = (uint32_t)pos;
        for (uint32_t L = 0; L < kLanes; L++) {
            const uint32_t nw = nwords[(uint64_t)b * kLanes + L];
            if (nw > 255 || pos + 4ull * nw + 64 > cap) return -1;
            hdr[(uint64_t)b * kHdrBytes + L] = (uint8_t)nw;
            pos += 4ull * nw;
        }
    }
    const uint64_t end = pos;

    // raw planes
    memset(low, 0, f.low_bytes(t | (lay << 4)));
    if (!lay) {
        parallel_range(f.M, 16, [&](uint64_t m0, uint64_t m1) {
            for (uint64_t m = m0; m < m1; m++) {
                if (t == kElemFp8) {
                    uint8_t *row = low + m * (f.K16 / 2);
                    for (uint32_t k = 0; k < f.K; k++) {
                        const uint32_t j = k & 15;   // nibble order: bytes 0..3 low = j 0..3, high = j 4..7, bytes 4..7 = j 8..15
                        row[(k >> 4) * 8 + (j & 3) + ((j >> 3) << 2)] |= (uint8_t)(S.low(m * K + k) << (((j >> 2) & 1) * 4));
                    }
                } else {
                    uint8_t *row = low + m * f.K16;
                    for (uint32_t k = 0; k < f.K; k++) row[k] = S.low(m * K + k);
                }
            }
        });
    }

    // pass 2: streams (and the layout 1 raw plane, in stream order) straight to their final offsets
    parallel_range(f.nb, 64, [&](uint64_t b0, uint64_t b1) {
        for (uint64_t b = b0; b < b1; b++) {
            const uint32_t rb = (uint32_t)(b / f.CB), cb = (uint32_t)(b % f.CB);
            const uint32_t nchunk = cb == f.CB - 1 ? f.nl : 32;
            const uint32_t npos = lay ? ((nchunk + 1) / 2) * 16 : kRows0 * 16;
            const uint64_t slot0 = (uint64_t)rb * f.spr + cb * 16;
            uint64_t off = bases[b];
            const uint64_t bend = b + 1 < f.nb ? bases[b + 1] : align8(end);
            for (uint32_t L = 0; L < kLanes; L++) {
                WordSink ws; ws.dst = data + off;
                for (uint32_t i = 0; i < npos; i++) {
                    LanePos p = lane_pos(lay, rb, cb, L, i);
                    if (p.row >= f.M || p.col >= f.K) { ws.put(2, 2); continue; }
                    const uint64_t wi = (uint64_t)p.row * K + p.col;
                    const uint8_t h = S.high(wi);
                    const uint32_t r = rank[h & 0x7F];
                    if (r < maxr) ws.put(2u | (h >> 7), (int)r + 2);     // r zeros, a one, the sign
                    else ws.put((1u << 8) | h, 24);                      // 15 zeros, a one, the whole byte
                    if (lay) {
                        const uint64_t o = (slot0 + (i >> 4)) * kLanes + L;
                        const uint32_t j = i & 15;
                        if (t == kElemFp8) low[o * 8 + 4 * ((j >> 3) & 1) + (j & 3)] |= (uint8_t)(S.low(wi) << (4 * ((j >> 2) & 1)));
                        else low[o * 16 + j] = S.low(wi);
                    }
                }
                ws.close();
                off += 4ull * ws.words;
            }
            for (uint64_t z = off; z < bend && z < cap; z++) data[z] = 0;   // alignment gap
        }
    });
    const uint64_t dl = align8(end) + 64;
    for (uint64_t z = end; z < dl && z < cap; z++) data[z] = 0;
    return (int64_t)dl;
}

// ---- layout 2 --------------------------------------------------------------------------------------------
int64_t encode_fixed(const Splitter &S, const void *wv, const Shape &f, uint64_t K, int t, uint16_t *psym,
                     uint32_t *bases, uint8_t *hdr, uint8_t *data, uint64_t cap, uint8_t *low) {
    const int nsym = t == kElemFp8 ? 20 : 128;
    const uint32_t esz = t == kElemFp8 ? 2 : 3;
    const uint64_t n = (uint64_t)f.M * K;
    const auto &T = fp8_tables();

    std::vector<std::array<uint64_t, 128>> part(host_threads() + 1);
    std::atomic<int> slot{0};
    parallel_range(n, 1u << 20, [&](uint64_t a, uint64_t b) {
        auto &h = part[slot++];
        h.fill(0);
        for (uint64_t i = a; i < b; i++) h[S.high(i) & 0x7F]++;
    });
    uint64_t hist[128] = {0};
    for (int s = 0; s < slot; s++) for (int k = 0; k < 128; k++) hist[k] += part[s][k];
    int ord[128];
    rank_symbols(hist, nsym, ord);
    uint8_t rank[128];
    for (int r = 0; r < 128; r++) rank[ord[r]] = (uint8_t)std::min(r, 7);
    for (uint32_t i = 0; i < kNpsym; i++) psym[i] = 0;
    for (int r = 0; r < 7; r++) {
        psym[r] = (uint16_t)(t == kElemFp8 ? T.hb2[ord[r]] : ord[r]);
        psym[8 + r] = (uint16_t)(t == kElemFp8 ? T.lb2[ord[r]] : 0);
    }

    auto each_pos = [&](uint32_t b, uint32_t L, auto &&fn) {
        const uint32_t rb = b / f.CB, cb = b % f.CB;
        const uint32_t nchunk = cb == f.CB - 1 ? f.nl : 32, nsc = (nchunk + 1) / 2;
        for (uint32_t i = 0; i < nsc * 16; i++) {
            const uint32_t sc = i >> 4, j = i & 15;
            const uint32_t row = rb * kRows12 + frag_row(L, j), col = cb * kCols + sc * 32 + frag_col(L, j);
            if (row >= f.M || col >= f.K) continue;
            fn(i, sc, j, (uint64_t)row * K + col);
        }
    };

    // exceptions per lane (uncapped)
    std::vector<uint32_t> cnt((size_t)f.nb * kLanes);
    parallel_range(f.nb, 64, [&](uint64_t b0, uint64_t b1) {
        for (uint64_t b = b0; b < b1; b++)
            for (uint32_t L = 0; L < kLanes; L++) {
                uint32_t c = 0;
                each_pos((uint32_t)b, L, [&](uint32_t, uint32_t, uint32_t, uint64_t wi) { c += rank[S.high(wi) & 0x7F] == 7; });
                cnt[b * kLanes + L] = c;
            }
    });

    // serial prefix with the reference's checks per exception (nwc_ops.cu:218-220): the 256th exception of a lane
    // is -3, an entry whose end + 64 passes the capacity is -1, whichever comes first in stream order
    uint64_t pos = 0;
    for (uint32_t b = 0; b < f.nb; b++) {
        pos = align8(pos);
        bases[b] = (uint32_t)pos;
        for (uint32_t L = 0; L < kLanes; L++) {
            const uint32_t c = cnt[(uint64_t)b * kLanes + L];
            const uint32_t upto = std::min<uint32_t>(c, 256);
            for (uint32_t k = 0; k < upto; k++) {      // first failing exception of this lane, if any
                if (k == 255) return -3;
                if (pos + (uint64_t)(k + 1) * esz + 64 > cap) return -1;
            }
            hdr[(uint64_t)b * kHdrBytes + L] = (uint8_t)c;
            pos += (uint64_t)c * esz;
        }
    }
    const uint64_t end = pos;

    const uint64_t nibb = f.nib2_bytes();
    memset(low, 0, nibb + f.raw2_bytes(t));
    uint8_t *nibp = low, *rawp = low + nibb;
    parallel_range(f.nb, 64, [&](uint64_t b0, uint64_t b1) {
        for (uint64_t b = b0; b < b1; b++) {
            const uint32_t rb = (uint32_t)(b / f.CB), cb = (uint32_t)(b % f.CB);
            const uint64_t slot0 = (uint64_t)rb * f.spr + cb * 16;
            uint64_t off = bases[b];
            for (uint32_t L = 0; L < kLanes; L++) {
                each_pos((uint32_t)b, L, [&](uint32_t i, uint32_t sc, uint32_t j, uint64_t wi) {
                    const uint8_t h = S.high(wi);
                    const uint32_t r = rank[h & 0x7F];
                    uint32_t v = S.low(wi);
                    if (r == 7) {                                   // exception: (index, value), planes stay zero
                        uint8_t *e = data + off;
                        e[0] = (uint8_t)i;
                        if (t == kElemFp8) e[1] = ((const uint8_t *)wv)[wi];
                        else { const uint16_t w = ((const uint16_t *)wv)[wi]; e[1] = (uint8_t)w; e[2] = (uint8_t)(w >> 8); }
                        off += esz;
                        v = 0;
                    }
                    nibp[((slot0 + sc) * kLanes + L) * 8 + (j >> 1)] |= (uint8_t)((((h >> 7) << 3) | r) << (4 * (j & 1)));
                    if (t == kElemFp8) {
                        // 32 three-bit fields per lane and super-chunk pair, field f at bit 3f of a 96-bit
                        // little-endian integer spread over words [pair][0..2][lane]
                        const uint32_t fld = 16 * (sc & 1) + j, bit = 3 * fld;
                        const uint64_t pair = (uint64_t)rb * f.spr2 + cb * 8 + (sc >> 1);
                        for (uint32_t k = bit >> 5; k <= (bit + 2) >> 5; k++) {
                            uint8_t *wp = rawp + ((pair * 3 + k) * kLanes + L) * 4;
                            uint32_t x; memcpy(&x, wp, 4);
                            const int sh = (int)bit - (int)(32 * k);
                            x |= sh >= 0 ? (v << sh) : (v >> -sh);
                            memcpy(wp, &x, 4);
                        }
                    } else {
                        rawp[((slot0 + sc) * kLanes + L) * 16 + j] = (uint8_t)v;
                    }
                });
            }
            const uint64_t bend = b + 1 < f.nb ? bases[b + 1] : align8(end);
            for (uint64_t z = off; z < bend && z < cap; z++) data[z] = 0;
        }
    });
    const uint64_t dl = align8(end) + 64;
    for (uint64_t z = end; z < dl && z < cap; z++) data[z] = 0;
    return (int64_t)dl;
}

}  // namespace

extern "C" int nwc_info(int what) {
    switch (what) {
        case 0: return kVersion;
        case 1: return 1;                  // states per lane
        case 2: return (int)kLutWords;     // table words
        case 3: return (int)kHdrBytes;     // header bytes per block
        case 4: return (int)kBlock;        // block size (fixed)
        case 5: return 1;                  // elem parameter on every entry point
        case 6: return 1;                  // layout 1
        case 7: return 1;                  // layout 2
        default: return -1;
    }
}

extern "C" int nwc_layout(uint64_t M, uint32_t K, int elem, uint64_t *out) {
    if (M == 0 || K == 0 || M > 0xFFFFFFFFull) return -1;
    Shape f((uint32_t)M, K, elem_layout(elem));
    out[0] = f.nb;
    out[1] = f.low_bytes(elem);
    out[2] = (uint64_t)f.Mp * f.CB;
    out[3] = f.K16;
    return 0;
}

extern "C" int64_t nwc_encode(const void *w, uint64_t n, uint32_t K, int elem, uint16_t *freq, uint16_t *psym,
                              uint32_t *bases, uint8_t *hdr, uint8_t *data, uint64_t data_cap, uint8_t *low) {
    if (K == 0 || n % K || n / K > 0xFFFFFFFFull) return -1;
    const int t = elem_type(elem), lay = elem_layout(elem);
    const uint64_t M = n / K;
    for (uint32_t i = 0; i < kNpsym; i++) freq[i] = 0;          // unused by format >= 9, cleared like the reference
    Splitter S{(const uint16_t *)w, (const uint8_t *)w, t == kElemFp8, lay == 2};
    if (t == kElemFp8) {                                         // NaN is rejected before anything is written
        std::atomic<bool> nan{false};
        const auto &T = fp8_tables();
        parallel_range(n, 1u << 20, [&](uint64_t a, uint64_t b) {
            for (uint64_t i = a; i < b && !nan.load(std::memory_order_relaxed); i++)
                if (T.sym01[((const uint8_t *)w)[i]] < 0) nan = true;
        });
        if (nan) return -2;
    }
    if (M == 0) return -1;
    Shape f((uint32_t)M, K, lay);
    if (lay == 2) return encode_fixed(S, w, f, K, t, psym, bases, hdr, data, data_cap, low);
    return encode_prefix(S, f, K, t, lay, psym, bases, hdr, data, data_cap, low);
}

// 4096-entry decode table of layouts 0/1: for every 12-bit window the codes that are complete inside it (at most
// two).  Two codes: c | b0 << 8 | b1 << 16 with c = bits of both.  Otherwise kFlag | (c of the first code, if
// complete) | b0 << 8 | (number of complete codes) << 24.  Entries 0 and 1 can never start with a complete code
// and carry exp_of_rank[11..14] instead (nwc_ops.cu:324-348).  Layout 2: words 0..1 = table byte of ranks 0..7,
// words 2..3 = low-byte bit 7 of ranks 0..7.
extern "C" void nwc_build_tab(const uint16_t *freq, const uint16_t *psym, int elem, uint32_t *lut) {
    (void)freq;
    if (elem_layout(elem) == 2) {
        memset(lut, 0, 4 * kLutWords);
        for (int r = 0; r < 8; r++) {
            lut[r / 4] |= (uint32_t)(psym[r] & 0xFF) << (8 * (r % 4));
            lut[2 + r / 4] |= (uint32_t)(psym[8 + r] & 0xFF) << (8 * (r % 4));
        }
        return;
    }
    const uint32_t maxr = elem_type(elem) == kElemFp8 ? kMaxRankFp8 : kMaxRankBf16;
    for (uint32_t pat = 0; pat < kLutWords; pat++) {
        uint32_t start = 0, got = 0, first_len = 0, bytes[2] = {0, 0};
        while (got < 2 && start < kPeek) {
            // leading zeros of the remaining window bits, counted inside the window only
            uint32_t z = 0;
            while (start + z < kPeek && !((pat >> (kPeek - 1 - start - z)) & 1)) z++;
            if (z >= maxr || start + z + 2 > kPeek) break;            // rank beyond the code, or not complete
            const uint32_t sign = (pat >> (kPeek - 1 - (start + z + 1))) & 1;
            bytes[got] = (sign << 7) | (psym[z] & 0x7F);
            start += z + 2;
            if (got++ == 0) first_len = start;
        }
        lut[pat] = got == 2 ? start | bytes[0] << 8 | bytes[1] << 16
                            : kFlag | (got ? first_len : 0u) | bytes[0] << 8 | got << 24;
    }
    lut[0] = kFlag | (uint32_t)(psym[11] & 0x7F) << 8 | (uint32_t)(psym[12] & 0x7F) << 16;
    lut[1] = kFlag | (uint32_t)(psym[13] & 0x7F) << 8 | (uint32_t)(psym[14] & 0x7F) << 16;
}

// Token-path decode table of layouts 0/1 with a 13-bit window, built from a stored LUT (its exp_of_rank): for every
// 13-bit window that starts with two complete codes, (16 - c) | b0 << 8 | b1 << 16, the step encoding of the gfx950
// kernel (byte 0 is the right shift that brings the second pair's 13 bits to [14:2] of its cursor's window, which
// starts one bit before the next code); for every other window the slow
// marker 0x40000000.  out[8192..8195] hold exp_of_rank[0..15] (the slow path's rank -> byte map).  Not part of the
// format: a 13-bit window makes a pair too long for the table 3-4x rarer than the stored 12-bit LUT does (0.025%
// instead of 0.087% of code pairs for N(0, 0.02^2) BF16), and each such pair costs its wave a code-by-code redo.
extern "C" int nwc_seq_table(const uint32_t *lut, int elem, uint32_t *out) {
    if (elem_layout(elem) > 1) return -1;
    const uint32_t maxr = elem_type(elem) == kElemFp8 ? kMaxRankFp8 : kMaxRankBf16;
    uint8_t eor[16] = {0};
    for (uint32_t q = 0; q < 15; q++) {                            // where lut_issue finds them (nwc_device.h)
        const uint32_t w = lut[q < 11u ? (1u << (kPeek - 1u - q)) : (q - 11u) >> 1];
        eor[q] = (uint8_t)((w >> ((q < 11u || (q & 1u)) ? 8u : 16u)) & 0x7Fu);
    }
    constexpr uint32_t P = kPeekSeq;
    for (uint32_t pat = 0; pat < (1u << P); pat++) {
        uint32_t start = 0, got = 0, bytes[2] = {0, 0};
        while (got < 2) {
            uint32_t z = 0;
            while (start + z < P && !((pat >> (P - 1 - start - z)) & 1)) z++;
            if (z >= maxr || start + z + 2 > P) break;
            const uint32_t sign = (pat >> (P - 1 - (start + z + 1))) & 1;
            bytes[got++] = (sign << 7) | eor[z];
            start += z + 2;
        }
        out[pat] = got == 2 ? (29u - P - start) | bytes[0] << 8 | bytes[1] << 16 : 0x40000000u;
    }
    for (uint32_t j = 0; j < 4; j++)
        out[(1u << P) + j] = eor[4 * j] | (uint32_t)eor[4 * j + 1] << 8 | (uint32_t)eor[4 * j + 2] << 16 |
                             (uint32_t)eor[4 * j + 3] << 24;
    return 0;
}
