/* nwc_oracle.c -- TEST INFRASTRUCTURE ONLY (see nwc_oracle.h).
 *
 * A deliberately literal, serial C restatement of the reference format.  It favours obviousness over speed:
 * the encoder walks blocks, lanes and stream positions in the reference's order with a bit accumulator, the
 * decoder reads one bit at a time.  The product library (nwc_amd/csrc) is written independently (parallel
 * encoder, word-window GPU decoders); the tests compare the two.
 */
#include "nwc_oracle.h"
#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { LANES = 32, COLS = 512, ROWS0 = 8, ROWS12 = 16, PEEK = 12, NLUT = 4096, HDRB = 32, NPSYM = 1024 };
enum { E_BF16 = 0, E_FP8 = 1 };
#define FLAGBIT (1u << 30)
#define TYPE(e) ((e) & 15)
#define LAYOUT(e) (((e) >> 4) & 15)

/* ---- Shape: nwc_ops.cu:87-98 ---- */
typedef struct { uint32_t M, K, K16, Kp, CB, Mp, nb, rows, nl, nsl, spr, nsl2, spr2; } shape_t;

static shape_t mk_shape(uint32_t M, uint32_t K, int layout) {
    shape_t s;
    s.M = M; s.K = K;
    s.rows = layout ? ROWS12 : ROWS0;
    s.K16 = (K + 15u) / 16u * 16u;
    s.CB = (K + COLS - 1) / COLS;
    s.Kp = s.CB * COLS;
    s.Mp = (M + s.rows - 1) / s.rows * s.rows;
    s.nb = (s.Mp / s.rows) * s.CB;
    s.nl = (s.K16 - (s.CB - 1) * COLS) / 16;      /* 16-column chunks coded in the last column block */
    s.nsl = (s.nl + 1) / 2;                       /* 32-column super-chunks there */
    s.spr = 16 * (s.CB - 1) + s.nsl;              /* super-chunk slots per 16-row group */
    s.nsl2 = (s.nsl + 1) / 2;
    s.spr2 = 8 * (s.CB - 1) + s.nsl2;             /* super-chunk pairs per row group (layout 2 fp8 raw plane) */
    return s;
}

/* ---- plane sizes: nwc_ops.cu:111-120 ---- */
static uint64_t nib_plane_bytes(const shape_t *s) { return (uint64_t)(s->Mp / 16) * s->spr * LANES * 8; }
static uint64_t raw_plane2_bytes(const shape_t *s, int t) {
    if (t == E_FP8) return (uint64_t)(s->Mp / 16) * s->spr2 * 3 * LANES * 4;
    return (uint64_t)(s->Mp / 16) * s->spr * LANES * 16;
}
static uint64_t low_bytes(const shape_t *s, int elem) {
    int t = TYPE(elem), lay = LAYOUT(elem);
    if (lay == 2) return nib_plane_bytes(s) + raw_plane2_bytes(s, t);
    if (lay) return (uint64_t)(s->Mp / 16) * s->spr * LANES * (t == E_FP8 ? 8 : 16);
    return t == E_FP8 ? (uint64_t)s->M * (s->K16 / 2) : (uint64_t)s->M * s->K16;
}

int or_layout(uint64_t M, uint32_t K, int elem, uint64_t *out) {
    if (M == 0 || K == 0 || M > 0xFFFFFFFFull) return -1;
    shape_t s = mk_shape((uint32_t)M, K, LAYOUT(elem));
    out[0] = s.nb; out[1] = low_bytes(&s, elem); out[2] = (uint64_t)s.Mp * s.CB; out[3] = s.K16;
    return 0;
}

/* ---- fp8 splits: nwc_ops.cu:140-148 (layouts 0/1) and :165-173 (layout 2) ---- */
static const uint8_t BYTE3_OF_SYM[10] = {60, 61, 62, 63, 64, 65, 66, 67, 59, 0};

int or_fp8_split(uint8_t b, uint8_t *sym, uint8_t *nib) {
    uint32_t e = (b >> 3) & 15u, m = b & 7u;
    if (e == 15 && m == 7) return -1;                               /* NaN */
    if (e >= 1) { *sym = (uint8_t)(e >> 1); *nib = (uint8_t)(((e & 1u) << 3) | m); return 0; }
    if (m >= 4) { *sym = 0; *nib = (uint8_t)((m - 4) << 1); return 0; }
    if (m == 0) { *sym = 9; *nib = 0; return 0; }
    *sym = 8; *nib = (uint8_t)(m == 1 ? 0 : (m == 2 ? 8 : 12));
    return 0;
}
int or_fp8_split2(uint8_t b, uint8_t *sym, uint8_t *m3) {
    uint32_t e = (b >> 3) & 15u, m = b & 7u;
    if (e == 15 && m == 7) return -1;
    if (e >= 1) { *sym = (uint8_t)e; *m3 = (uint8_t)m; return 0; }
    if (m >= 4) { *sym = 16; *m3 = (uint8_t)((m - 4) << 1); return 0; }
    if (m >= 2) { *sym = 17; *m3 = (uint8_t)((m - 2) << 2); return 0; }
    *sym = (uint8_t)(m == 1 ? 18 : 19); *m3 = 0;
    return 0;
}
uint8_t or_fp8_hb2(int sym) {
    if (sym >= 1 && sym <= 15) return (uint8_t)(60 + (sym >> 1));   /* fp32 exponent (120 + e) >> 1 */
    if (sym == 16) return 60;
    if (sym == 17 || sym == 18) return 59;
    return 0;
}
uint8_t or_fp8_lb2(int sym) {
    if (sym >= 1 && sym <= 15) return (uint8_t)((sym & 1) << 7);    /* the exponent's low bit */
    return (uint8_t)(sym == 17 ? 0x80 : 0);
}

/* layout 0 fp8 nibble position of column j (0..15) of a lane: nwc_ops.cu:151-152 */
static uint32_t nib_byte0(uint32_t j) { return (j & 3u) + ((j >> 3) << 2); }
static uint32_t nib_shift0(uint32_t j) { return ((j >> 2) & 1u) * 4u; }

/* ---- fragment order: nwc_ops.cu:159-160, docs/format.md 4c ---- */
uint32_t or_frag_row(uint32_t lane, uint32_t i) { return (lane >> 2) + 8u * ((i >> 1) & 1u); }
uint32_t or_frag_col(uint32_t lane, uint32_t i) {
    return 8u * (lane & 3u) + 4u * ((i >> 3) & 1u) + 2u * ((i >> 2) & 1u) + (i & 1u);
}

/* ---- symbol ranking: nwc_ops.cu:193-194 / :275-277 (exchange sort, NOT stable) ---- */
static void rank_symbols(const uint8_t *high, uint64_t n, int nsym, int ord[128]) {
    uint64_t hist[128];
    memset(hist, 0, sizeof hist);
    for (uint64_t i = 0; i < n; i++) hist[high[i] & 0x7F]++;
    for (int i = 0; i < 128; i++) ord[i] = i;
    for (int a = 0; a < nsym; a++)
        for (int b = a + 1; b < nsym; b++)
            if (hist[ord[b]] > hist[ord[a]]) { int t = ord[a]; ord[a] = ord[b]; ord[b] = t; }
}

/* ---- MSB-first bit sink into 32-bit words (nwc_ops.cu:129-133) ---- */
typedef struct { uint32_t *w; uint32_t nw; uint64_t acc; int nacc; } bitsink_t;
static void put_bits(bitsink_t *b, uint32_t v, int nbits) {
    for (int k = nbits - 1; k >= 0; k--) {
        b->acc = (b->acc << 1) | ((v >> k) & 1u);
        if (++b->nacc == 32) { b->w[b->nw++] = (uint32_t)b->acc; b->acc = 0; b->nacc = 0; }
    }
}
static void flush_bits(bitsink_t *b) {
    if (b->nacc) { b->w[b->nw++] = (uint32_t)(b->acc << (32 - b->nacc)); b->acc = 0; b->nacc = 0; }
}
static void store_le32(uint8_t *p, uint32_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); p[2] = (uint8_t)(v >> 16); p[3] = (uint8_t)(v >> 24); }
static uint32_t load_le32(const uint8_t *p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }
static uint64_t align8(uint64_t v) { return (v + 7) / 8 * 8; }

/* split every weight into (symbol | sign << 7, raw byte / nibble / 3-bit field) */
static int split_weights(const void *wv, uint64_t n, int t, int lay, uint8_t *high, uint8_t *raw) {
    for (uint64_t i = 0; i < n; i++) {
        if (t == E_FP8) {
            uint8_t b = ((const uint8_t *)wv)[i], sym, r;
            int bad = (lay == 2) ? or_fp8_split2(b, &sym, &r) : or_fp8_split(b, &sym, &r);
            if (bad) return -2;
            high[i] = (uint8_t)((b & 0x80u) | sym); raw[i] = r;
        } else {
            uint16_t v = ((const uint16_t *)wv)[i];
            high[i] = (uint8_t)(v >> 8); raw[i] = (uint8_t)v;
        }
    }
    return 0;
}

/* ---- layout 2 encoder: nwc_ops.cu:175-243 ---- */
static int64_t encode_l2(const void *wv, uint64_t n, uint32_t K, int t, uint16_t *psym, uint32_t *bases,
                         uint8_t *hdr, uint8_t *data, uint64_t cap, uint8_t *low) {
    shape_t s = mk_shape((uint32_t)(n / K), K, 2);
    const int nsym = t == E_FP8 ? 20 : 128, esz = t == E_FP8 ? 2 : 3;
    uint8_t *high = (uint8_t *)malloc(n ? n : 1), *raw = (uint8_t *)malloc(n ? n : 1);
    int64_t rc = -1;
    if (split_weights(wv, n, t, 2, high, raw)) { rc = -2; goto out; }
    int ord[128]; rank_symbols(high, n, nsym, ord);
    uint8_t rank[128];
    for (int r = 0; r < 128; r++) rank[ord[r]] = (uint8_t)(r < 7 ? r : 7);
    for (int i = 0; i < NPSYM; i++) psym[i] = 0;
    for (int r = 0; r < 7; r++) {
        psym[r] = (uint16_t)(t == E_FP8 ? or_fp8_hb2(ord[r]) : ord[r]);
        psym[8 + r] = (uint16_t)(t == E_FP8 ? or_fp8_lb2(ord[r]) : 0);
    }
    uint64_t nibb = nib_plane_bytes(&s);
    memset(low, 0, nibb + raw_plane2_bytes(&s, t));
    uint8_t *nibp = low, *rawp = low + nibb;
    uint64_t pos = 0;
    for (uint32_t b = 0; b < s.nb; b++) {
        uint32_t rb = b / s.CB, cb = b % s.CB;
        uint32_t nchunk = cb == s.CB - 1 ? s.nl : 32, nsc = (nchunk + 1) / 2, slot0 = rb * s.spr + cb * 16;
        uint64_t p8 = align8(pos);
        if (p8 > cap) goto out;
        for (uint64_t z = pos; z < p8; z++) data[z] = 0;
        pos = p8; bases[b] = (uint32_t)pos;
        for (uint32_t L = 0; L < LANES; L++) {
            uint32_t cnt = 0;
            for (uint32_t i = 0; i < nsc * 16; i++) {
                uint32_t sc = i >> 4, j = i & 15;
                uint32_t row = rb * 16 + or_frag_row(L, j), col = cb * COLS + sc * 32 + or_frag_col(L, j);
                if (row >= s.M || col >= s.K) continue;              /* filler: nibble 0, raw 0 */
                uint64_t wi = (uint64_t)row * K + col;
                uint32_t sg = high[wi] >> 7, r = rank[high[wi] & 0x7F];
                uint8_t v = raw[wi];
                if (r == 7) {                                       /* exception entry (index, value) */
                    if (cnt == 255) { rc = -3; goto out; }
                    if (pos + (uint64_t)cnt * esz + esz + 64 > cap) { rc = -1; goto out; }
                    uint8_t *e = data + pos + (uint64_t)cnt * esz;
                    e[0] = (uint8_t)i;
                    if (t == E_FP8) e[1] = ((const uint8_t *)wv)[wi];
                    else { uint16_t w = ((const uint16_t *)wv)[wi]; e[1] = (uint8_t)w; e[2] = (uint8_t)(w >> 8); }
                    v = 0; cnt++;
                }
                nibp[((uint64_t)(slot0 + sc) * LANES + L) * 8 + (j >> 1)] |= (uint8_t)(((sg << 3) | r) << (4 * (j & 1)));
                if (t == E_FP8) {
                    uint32_t tt = 16 * (sc & 1) + j, bit = 3 * tt, k = bit >> 5, sh = bit & 31;
                    uint64_t pair = (uint64_t)rb * s.spr2 + cb * 8 + (sc >> 1);
                    uint8_t *w0 = rawp + ((pair * 3 + k) * LANES + L) * 4;
                    store_le32(w0, load_le32(w0) | ((uint32_t)v << sh));
                    if (sh > 29) { uint8_t *w1 = w0 + LANES * 4; store_le32(w1, load_le32(w1) | ((uint32_t)v >> (32 - sh))); }
                } else {
                    rawp[((uint64_t)(slot0 + sc) * LANES + L) * 16 + j] = v;
                }
            }
            hdr[(uint64_t)b * HDRB + L] = (uint8_t)cnt;
            pos += (uint64_t)cnt * esz;
        }
    }
    {
        uint64_t end = align8(pos) + 64;
        if (end > cap) end = cap;
        for (uint64_t z = pos; z < end; z++) data[z] = 0;
    }
    rc = (int64_t)(align8(pos) + 64);
out:
    free(high); free(raw);
    return rc;
}

/* ---- layouts 0/1 encoder: nwc_ops.cu:245-320 ---- */
int64_t or_encode(const void *wv, uint64_t n, uint32_t K, int elem, uint16_t *freq, uint16_t *psym,
                  uint32_t *bases, uint8_t *hdr, uint8_t *data, uint64_t cap, uint8_t *low) {
    if (K == 0 || n % K || n / K > 0xFFFFFFFFull) return -1;
    const int t = TYPE(elem), lay = LAYOUT(elem);
    if (lay == 2) {
        for (int i = 0; i < NPSYM; i++) freq[i] = 0;
        return encode_l2(wv, n, K, t, psym, bases, hdr, data, cap, low);
    }
    shape_t s = mk_shape((uint32_t)(n / K), K, lay);
    const int nsym = t == E_FP8 ? 10 : 128, maxr = t == E_FP8 ? 10 : 15;
    uint8_t *high = (uint8_t *)malloc(n ? n : 1), *raw = (uint8_t *)malloc(n ? n : 1);
    int64_t rc = -1;
    if (split_weights(wv, n, t, lay, high, raw)) { rc = -2; goto out; }
    memset(low, 0, low_bytes(&s, elem));
    if (!lay) {                                    /* row-major raw plane, stride K16 (fp8: K16/2 bytes of nibbles) */
        for (uint32_t m = 0; m < s.M; m++)
            for (uint32_t k = 0; k < s.K; k++) {
                uint8_t v = raw[(uint64_t)m * K + k];
                if (t == E_FP8) low[(uint64_t)m * (s.K16 / 2) + (k / 16) * 8 + nib_byte0(k & 15)] |= (uint8_t)(v << nib_shift0(k & 15));
                else low[(uint64_t)m * s.K16 + k] = v;
            }
    }
    int ord[128]; rank_symbols(high, n, nsym, ord);
    uint8_t rank[128];
    for (int r = 0; r < 128; r++) rank[ord[r]] = (uint8_t)r;
    for (int i = 0; i < NPSYM; i++) {
        freq[i] = 0;
        psym[i] = 0;
        if (i < 16) psym[i] = (uint16_t)(t == E_FP8 ? (i < 10 ? BYTE3_OF_SYM[ord[i]] : 0) : ord[i]);
    }
    uint32_t words[(2 * ROWS0 * COLS) / LANES + 2 + 64];
    uint64_t pos = 0;
    for (uint32_t b = 0; b < s.nb; b++) {
        uint32_t rb = b / s.CB, cb = b % s.CB;
        uint32_t nchunk = cb == s.CB - 1 ? s.nl : 32, slot0 = rb * s.spr + cb * 16;
        uint64_t p8 = align8(pos);
        if (p8 > cap) goto out;
        for (uint64_t z = pos; z < p8; z++) data[z] = 0;
        pos = p8; bases[b] = (uint32_t)pos;
        for (uint32_t L = 0; L < LANES; L++) {
            bitsink_t bs = {words, 0, 0, 0};
            uint32_t nw = lay ? ((nchunk + 1) / 2) * 16 : ROWS0 * 16;
            for (uint32_t i = 0; i < nw; i++) {
                uint32_t row, col;
                if (lay) { row = rb * 16 + or_frag_row(L, i & 15); col = cb * COLS + (i >> 4) * 32 + or_frag_col(L, i & 15); }
                else     { row = rb * ROWS0 + (i >> 4); col = cb * COLS + L * 16 + (i & 15); }
                if (row >= s.M || col >= s.K) { put_bits(&bs, 2, 2); continue; }   /* filler "10": rank 0, + */
                uint64_t wi = (uint64_t)row * K + col;
                uint8_t e = high[wi];
                uint32_t r = rank[e & 0x7F], sg = e >> 7;
                if ((int)r < maxr) { put_bits(&bs, 1, (int)r + 1); put_bits(&bs, sg, 1); }
                else { put_bits(&bs, 1, 16); put_bits(&bs, e, 8); }      /* escape (BF16 only) */
                if (lay) {
                    uint64_t o = (uint64_t)(slot0 + (i >> 4)) * LANES + L;
                    uint32_t j = i & 15;
                    if (t == E_FP8) low[o * 8 + 4 * ((j >> 3) & 1) + (j & 3)] |= (uint8_t)(raw[wi] << (4 * ((j >> 2) & 1)));
                    else low[o * 16 + j] = raw[wi];
                }
            }
            flush_bits(&bs);
            if (bs.nw > 255 || pos + 4ull * bs.nw + 64 > cap) goto out;
            hdr[(uint64_t)b * HDRB + L] = (uint8_t)bs.nw;
            for (uint32_t k = 0; k < bs.nw; k++) store_le32(data + pos + 4ull * k, words[k]);
            pos += 4ull * bs.nw;
        }
    }
    {
        uint64_t end = align8(pos) + 64;
        if (end > cap) end = cap;
        for (uint64_t z = pos; z < end; z++) data[z] = 0;
    }
    rc = (int64_t)(align8(pos) + 64);
out:
    free(high); free(raw);
    return rc;
}

/* ---- lookup table: nwc_ops.cu:324-348 ---- */
static uint32_t lead0(uint32_t x) { uint32_t u = 0; if (!x) return 32; while (!(x & 0x80000000u)) { x <<= 1; u++; } return u; }

void or_build_tab(const uint16_t *psym, int elem, uint32_t *lut) {
    if (LAYOUT(elem) == 2) {
        memset(lut, 0, 4 * NLUT);
        for (int r = 0; r < 8; r++) {
            lut[r >> 2] |= (uint32_t)(psym[r] & 0xFFu) << (8 * (r & 3));
            lut[2 + (r >> 2)] |= (uint32_t)(psym[8 + r] & 0xFFu) << (8 * (r & 3));
        }
        return;
    }
    const uint32_t maxr = TYPE(elem) == E_FP8 ? 10 : 15;
    for (uint32_t pat = 0; pat < NLUT; pat++) {
        uint32_t bits = pat << (32 - PEEK), used = 0, ncode = 0, c1 = 0, by[2] = {0, 0};
        for (int k = 0; k < 2; k++) {
            uint32_t left = PEEK - used;
            if (left == 0) break;
            uint32_t x = bits << used, u = lead0(x);
            if (u >= maxr || u + 2 > left) break;
            uint32_t sg = (x >> (30 - u)) & 1u;
            by[k] = (sg << 7) | (psym[u] & 0x7Fu);
            used += u + 2; ncode++;
            if (k == 0) c1 = used;
        }
        if (ncode == 2) lut[pat] = used | (by[0] << 8) | (by[1] << 16);
        else lut[pat] = FLAGBIT | (ncode ? c1 : 0u) | (by[0] << 8) | (ncode << 24);
    }
    lut[0] = FLAGBIT | ((psym[11] & 0x7Fu) << 8) | ((psym[12] & 0x7Fu) << 16);
    lut[1] = FLAGBIT | ((psym[13] & 0x7Fu) << 8) | ((psym[14] & 0x7Fu) << 16);
}

/* ---- bit-serial decoder (test_format_cpu.py:22-73) ---- */
typedef struct { const uint8_t *base; uint64_t off, len, nbits, pos; } bitsrc_t;   /* len: bytes available */
static int get_bit(bitsrc_t *b, uint32_t *v) {
    if (b->pos >= b->nbits) return -1;
    uint64_t w = b->pos >> 5; uint32_t k = (uint32_t)(b->pos & 31);
    if (b->off + 4 * w + 4 > b->len) return -1;
    *v = (load_le32(b->base + b->off + 4 * w) >> (31 - k)) & 1u;
    b->pos++;
    return 0;
}

/* exp_of_rank read back from the table (test_format_cpu.py:14-19) */
static void ranks_from_lut(const uint32_t *lut, uint8_t eor[16]) {
    for (int r = 0; r < 11; r++) eor[r] = (uint8_t)((lut[1u << (PEEK - 1 - r)] >> 8) & 0x7F);
    eor[11] = (uint8_t)((lut[0] >> 8) & 0x7F); eor[12] = (uint8_t)((lut[0] >> 16) & 0x7F);
    eor[13] = (uint8_t)((lut[1] >> 8) & 0x7F); eor[14] = (uint8_t)((lut[1] >> 16) & 0x7F);
    eor[15] = 0;
}

/* one row group (all column blocks) of layouts 0/1 into tile[rows x K] (BF16 bits; rows beyond M ignored) */
static int decode_group01(const uint8_t *data, uint64_t dlen, const uint32_t *bases, const uint8_t *hdr, const uint8_t *eor,
                          const uint8_t *low, const shape_t *s, int t, int lay, uint32_t rb, uint16_t *tile) {
    const uint32_t maxr = t == E_FP8 ? 10 : 15;
    for (uint32_t cb = 0; cb < s->CB; cb++) {
        uint32_t b = rb * s->CB + cb;
        uint32_t nchunk = cb == s->CB - 1 ? s->nl : 32, slot0 = rb * s->spr + cb * 16;
        uint64_t off = bases[b];
        for (uint32_t L = 0; L < LANES; L++) {
            uint32_t nwords = hdr[(uint64_t)b * HDRB + L];
            bitsrc_t bs = {data, off, dlen, 32ull * nwords, 0};
            off += 4ull * nwords;
            uint32_t nw = lay ? ((nchunk + 1) / 2) * 16 : ROWS0 * 16;
            for (uint32_t i = 0; i < nw; i++) {
                uint32_t row, col, j = i & 15;
                if (lay) { row = rb * 16 + or_frag_row(L, j); col = cb * COLS + (i >> 4) * 32 + or_frag_col(L, j); }
                else     { row = rb * ROWS0 + (i >> 4); col = cb * COLS + L * 16 + j; }
                uint32_t zeros = 0, bit, e, sg = 0, esc = 0;
                for (;;) { if (get_bit(&bs, &bit)) return -1; if (bit) break; zeros++; if (zeros > 15) return -1; }
                if (zeros < maxr) {
                    if (get_bit(&bs, &sg)) return -1;
                    e = (sg << 7) | eor[zeros];
                } else {
                    if (t == E_FP8) return -1;
                    e = 0; esc = 1;
                    for (int k = 0; k < 8; k++) { if (get_bit(&bs, &bit)) return -1; e = (e << 1) | bit; }
                }
                if (row >= s->M || col >= s->K) {
                    if (zeros != 0 || sg != 0 || esc) return -2;          /* fillers are "10" */
                    continue;
                }
                uint32_t lowbits;
                if (!lay) {
                    if (t == E_FP8) lowbits = (low[(uint64_t)row * (s->K16 / 2) + (col / 16) * 8 + nib_byte0(col & 15)] >> nib_shift0(col & 15)) & 15u;
                    else lowbits = low[(uint64_t)row * s->K16 + col];
                } else {
                    uint64_t o = (uint64_t)(slot0 + (i >> 4)) * LANES + L;
                    if (t == E_FP8) lowbits = (low[o * 8 + 4 * ((j >> 3) & 1) + (j & 3)] >> (4 * ((j >> 2) & 1))) & 15u;
                    else lowbits = low[o * 16 + j];
                }
                /* BF16: [sign | 7-bit exponent byte][raw byte].  fp8: the fp32 pattern [s | byte3][nibble << 4][0][0]
                   (docs/format.md 4b), whose upper half is the BF16 of the unscaled fp8 value. */
                uint16_t v = t == E_FP8 ? (uint16_t)((e << 8) | (lowbits << 4)) : (uint16_t)((e << 8) | lowbits);
                tile[(uint64_t)(row - rb * s->rows) * s->K + col] = v;
            }
        }
    }
    return 0;
}

static uint16_t bf16_rne(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40);   /* quiet NaN */
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* layout 2 (test_format_cpu.py:76-111; fp8 raw fields nwc_ops.cu:228-233, values :866-870) */
static int decode_group2(const uint8_t *data, uint64_t dlen, const uint32_t *bases, const uint8_t *hdr, const uint32_t *lut,
                         const uint8_t *low, const shape_t *s, int t, uint32_t rb, uint16_t *tile) {
    const uint32_t esz = t == E_FP8 ? 2 : 3;
    uint8_t hb[8], lb[8];
    for (int r = 0; r < 8; r++) { hb[r] = (uint8_t)(lut[r >> 2] >> (8 * (r & 3))); lb[r] = (uint8_t)(lut[2 + (r >> 2)] >> (8 * (r & 3))); }
    const uint8_t *nibp = low, *rawp = low + nib_plane_bytes(s);
    for (uint32_t cb = 0; cb < s->CB; cb++) {
        uint32_t b = rb * s->CB + cb;
        uint32_t nchunk = cb == s->CB - 1 ? s->nl : 32, nsc = (nchunk + 1) / 2, slot0 = rb * s->spr + cb * 16;
        uint64_t off = bases[b];
        for (uint32_t L = 0; L < LANES; L++) {
            uint32_t cnt = hdr[(uint64_t)b * HDRB + L];
            if (off + (uint64_t)cnt * esz > dlen) return -1;
            const uint8_t *ent = data + off;
            off += (uint64_t)cnt * esz;
            uint8_t used[256];
            memset(used, 0, sizeof used);
            for (uint32_t i = 0; i < nsc * 16; i++) {
                uint32_t sc = i >> 4, j = i & 15;
                uint32_t row = rb * 16 + or_frag_row(L, j), col = cb * COLS + sc * 32 + or_frag_col(L, j);
                uint64_t slot = (uint64_t)(slot0 + sc) * LANES + L;
                uint32_t nib = (nibp[slot * 8 + (j >> 1)] >> (4 * (j & 1))) & 15u, sg = nib >> 3, rk = nib & 7;
                uint32_t field;
                if (t == E_FP8) {
                    uint32_t tt = 16 * (sc & 1) + j, bit = 3 * tt;
                    uint64_t pair = (uint64_t)rb * s->spr2 + cb * 8 + (sc >> 1);
                    uint64_t w96 = 0; uint32_t w2;
                    w96 = (uint64_t)load_le32(rawp + ((pair * 3 + 0) * LANES + L) * 4) |
                          ((uint64_t)load_le32(rawp + ((pair * 3 + 1) * LANES + L) * 4) << 32);
                    w2 = load_le32(rawp + ((pair * 3 + 2) * LANES + L) * 4);
                    if (bit < 64) field = (uint32_t)((w96 >> bit) & 7u) | (bit > 61 ? (uint32_t)((w2 << (64 - bit)) & 7u) : 0u);
                    else field = (w2 >> (bit - 64)) & 7u;
                } else field = rawp[slot * 16 + j];
                if (row >= s->M || col >= s->K) { if (nib || field) return -3; continue; }
                uint16_t v;
                if (rk == 7) {                                        /* exception: planes zero, value in the entry list */
                    if (field) return -3;
                    int found = -1;
                    for (uint32_t k = 0; k < cnt; k++) if (ent[k * esz] == i) { if (found >= 0) return -4; found = (int)k; }
                    if (found < 0) return -4;
                    used[found] = 1;
                    const uint8_t *e = ent + (uint64_t)found * esz;
                    if (t == E_FP8) v = bf16_rne(or_e4m3_to_f32(e[1]));
                    else v = (uint16_t)(e[1] | (e[2] << 8));
                } else if (t == E_FP8) v = (uint16_t)((sg << 15) | ((uint32_t)hb[rk] << 8) | lb[rk] | (field << 4));
                else v = (uint16_t)((sg << 15) | ((uint32_t)hb[rk] << 8) | field);
                tile[(uint64_t)(row - rb * 16) * s->K + col] = v;
            }
            for (uint32_t k = 0; k < cnt; k++) if (!used[k]) return -4;
        }
    }
    return 0;
}

static int decode_group(const uint8_t *data, uint64_t dlen, const uint32_t *bases, const uint8_t *hdr, const uint32_t *lut,
                        const uint8_t *low, const shape_t *s, int elem, uint32_t rb, uint16_t *tile) {
    int t = TYPE(elem), lay = LAYOUT(elem);
    if (lay == 2) return decode_group2(data, dlen, bases, hdr, lut, low, s, t, rb, tile);
    uint8_t eor[16]; ranks_from_lut(lut, eor);
    return decode_group01(data, dlen, bases, hdr, eor, low, s, t, lay, rb, tile);
}

int or_decode(const uint8_t *data, uint64_t dlen, const uint32_t *bases, const uint8_t *hdr, const uint32_t *lut,
              const uint8_t *low, uint64_t M, uint32_t K, int elem, uint16_t *out, int threads) {
    if (M == 0 || K == 0 || M > 0xFFFFFFFFull) return -5;
    int lay = LAYOUT(elem);
    if (lay > 2 || TYPE(elem) > 1) return -5;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    shape_t s = mk_shape((uint32_t)M, K, lay);
    int rc = 0;
    uint32_t ngroups = s.Mp / s.rows;
    #pragma omp parallel
    {
        uint16_t *tile = (uint16_t *)malloc((size_t)s.rows * K * 2);
        #pragma omp for schedule(dynamic, 4)
        for (int64_t g = 0; g < (int64_t)ngroups; g++) {
            int r = decode_group(data, dlen, bases, hdr, lut, low, &s, elem, (uint32_t)g, tile);
            if (r) {
                #pragma omp critical
                rc = rc ? rc : r;
                continue;
            }
            for (uint32_t rr = 0; rr < s.rows; rr++) {
                uint64_t row = (uint64_t)g * s.rows + rr;
                if (row < M) memcpy(out + row * K, tile + (uint64_t)rr * K, (size_t)K * 2);
            }
        }
        free(tile);
    }
    return rc;
}

/* ---- fp32 matvec on BF16 weights ---- */
static float bf16_to_f32(uint16_t h) { uint32_t u = (uint32_t)h << 16; float f; memcpy(&f, &u, 4); return f; }

static float dot_row(const uint16_t *w, const float *x, uint32_t K) {
    float acc = 0.f;
    for (uint32_t k = 0; k < K; k++) acc += bf16_to_f32(w[k]) * x[k];
    return acc;
}

void or_matvec_f32(const uint16_t *w, uint64_t M, uint32_t K, const float *x, float *y, int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    #pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < (int64_t)M; m++) y[m] = dot_row(w + (uint64_t)m * K, x, K);
}

int or_linear(const uint8_t *data, uint64_t dlen, const uint32_t *bases, const uint8_t *hdr, const uint32_t *lut,
              const uint8_t *low, uint64_t M, uint32_t K, int elem, const float *x, const float *scale, float *y,
              int threads) {
    if (M == 0 || K == 0 || M > 0xFFFFFFFFull) return -5;
    int lay = LAYOUT(elem);
    if (lay > 2 || TYPE(elem) > 1) return -5;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    shape_t s = mk_shape((uint32_t)M, K, lay);
    uint32_t ngroups = s.Mp / s.rows;
    int rc = 0;
    #pragma omp parallel
    {
        uint16_t *tile = (uint16_t *)malloc((size_t)s.rows * K * 2);
        #pragma omp for schedule(dynamic, 4)
        for (int64_t g = 0; g < (int64_t)ngroups; g++) {
            int r = decode_group(data, dlen, bases, hdr, lut, low, &s, elem, (uint32_t)g, tile);
            if (r) {
                #pragma omp critical
                rc = rc ? rc : r;
                continue;
            }
            for (uint32_t rr = 0; rr < s.rows; rr++) {
                uint64_t row = (uint64_t)g * s.rows + rr;
                if (row >= M) break;
                float v = dot_row(tile + (uint64_t)rr * K, x, K);
                y[row] = scale ? v * scale[row] : v;
            }
        }
        free(tile);
    }
    return rc;
}

/* ---- fp8 e4m3fn from the definition ---- */
float or_e4m3_to_f32(uint8_t b) {
    uint32_t sg = b >> 7, e = (b >> 3) & 15u, m = b & 7u;
    float v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = (float)m * (1.0f / 512.0f);
    else v = ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
    return sg ? -v : v;
}

uint8_t or_f32_to_e4m3(float v) {
    uint8_t sg = signbit(v) ? 0x80 : 0;
    double a = fabs((double)v);
    if (isnan(v)) return 0x7F;
    if (a > 448.0) a = 448.0;
    /* candidates are the 127 non-negative finite codes; pick the nearest, ties to the even code */
    uint8_t best = 0; double bd = 1e300;
    for (uint32_t c = 0; c < 127; c++) {
        double cv = (double)or_e4m3_to_f32((uint8_t)c), d = fabs(cv - a);
        if (d < bd || (d == bd && (c & 1) == 0 && (best & 1))) { bd = d; best = (uint8_t)c; }
    }
    return (uint8_t)(sg | best);
}

void or_quantize_e4m3(const float *v, uint64_t n, uint8_t *out, int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; i++) out[i] = or_f32_to_e4m3(v[i]);
}
