// Host sanitizer run (AddressSanitizer + UndefinedBehaviorSanitizer) of the library's encoder
// (nwc_amd/csrc/encode.cpp: nwc_encode, nwc_build_tab, nwc_seq_table, nwc_layout) and of the C oracle
// (oracle/nwc_oracle.c) on the encoder test cases of tests/test_encoder.py: N(0, sigma^2) and exponent-spread BF16
// matrices and fp8 matrices in layouts 0, 1 and 2, including ragged shapes (K = 40, 4097, 1000) and matrices large
// enough for the encoder's threads to split the work.  For every case both encoders' outputs are compared byte for
// byte, both decode tables are compared, and the oracle decodes the stream back to the input.  Exit status 0 and
// "selftest: N cases ok" on success; a sanitizer report aborts the run (halt_on_error).  Test infrastructure only.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

extern "C" {
#include "nwc_oracle.h"
}
#include "nwc_ops.h"

namespace {

// freq/psym of 1024 entries, 32 header bytes per block, the 4096-word table, the 13-bit table, raw-plane slack
constexpr int kNpair = 1024, kLanes = 32, kTabWords = 4096, kSeqWords = 8196, kRawSlack = 512;

struct Rng {
    uint64_t s;
    uint64_t next() {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return s * 2685821657736338717ull;
    }
    double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
    double normal() { return std::sqrt(-2.0 * std::log(uniform())) * std::cos(6.283185307179586 * uniform()); }
};

uint16_t bf16_rne(float v) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

uint16_t bf16_of_e4m3(uint8_t b) {
    const float f = or_e4m3_to_f32(b);
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return (uint16_t)(u >> 16);                               // exact: e4m3 has 3 mantissa bits
}

struct Encoded {
    int64_t dl = -1;
    std::vector<uint16_t> freq, psym;
    std::vector<uint32_t> bases, lut;
    std::vector<uint8_t> hdr, data, low;
};

template <class Enc>
Encoded run_encoder(Enc enc, const void *w, uint64_t M, uint32_t K, int elem, const uint64_t info[4]) {
    const uint64_t n = M * K, nb = info[0];
    Encoded e;
    e.freq.assign(kNpair, 0);
    e.psym.assign(kNpair, 0);
    e.bases.assign(nb, 0);
    e.hdr.assign(nb * kLanes, 0);
    e.low.assign(info[1] + kRawSlack, 0);
    for (uint64_t cap : {n + n / 2 + nb * 64 + 4096, 3 * n + nb * 64 + 4096}) {
        e.data.assign(cap, 0);
        e.dl = enc(w, n, K, elem, e.freq.data(), e.psym.data(), e.bases.data(), e.hdr.data(), e.data.data(), cap,
                   e.low.data());
        if (e.dl >= 0 || e.dl == -2 || e.dl == -3) break;
    }
    return e;
}

int fail(const char *what, uint64_t M, uint32_t K, int elem) {
    std::fprintf(stderr, "selftest: %s differs (M=%llu K=%u elem=0x%x)\n", what, (unsigned long long)M, K, elem);
    return 1;
}

// One case: both encoders, both tables, the oracle's decode against the input.
int check(const void *w, const std::vector<uint16_t> &expect, uint64_t M, uint32_t K, int elem) {
    uint64_t info[4], oinfo[4];
    if (nwc_layout(M, K, elem, info) != 0 || or_layout(M, K, elem, oinfo) != 0) return fail("layout call", M, K, elem);
    if (std::memcmp(info, oinfo, sizeof info) != 0) return fail("layout", M, K, elem);
    const Encoded a = run_encoder(nwc_encode, w, M, K, elem, info);
    const Encoded b = run_encoder(or_encode, w, M, K, elem, info);
    if (a.dl < 0 || a.dl != b.dl) return fail("data length", M, K, elem);
    const size_t dl = (size_t)a.dl;
    if (std::memcmp(a.data.data(), b.data.data(), dl) != 0) return fail("data", M, K, elem);
    if (a.bases != b.bases) return fail("bases", M, K, elem);
    if (a.hdr != b.hdr) return fail("hdr", M, K, elem);
    if (std::memcmp(a.low.data(), b.low.data(), info[1]) != 0) return fail("raw plane", M, K, elem);
    if (a.psym != b.psym) return fail("psym", M, K, elem);
    std::vector<uint32_t> lut_a(kTabWords, 0), lut_b(kTabWords, 0);
    nwc_build_tab(a.freq.data(), a.psym.data(), elem, lut_a.data());
    or_build_tab(b.psym.data(), elem, lut_b.data());
    if (lut_a != lut_b) return fail("decode table", M, K, elem);
    if (((elem >> 4) & 15) <= 1) {
        std::vector<uint32_t> seq(kSeqWords, 0);
        if (nwc_seq_table(lut_a.data(), elem, seq.data()) != 0) return fail("13-bit table call", M, K, elem);
    }
    std::vector<uint8_t> stored(dl + 64, 0);                 // the data tensor: the stream plus 64 zero bytes
    std::memcpy(stored.data(), a.data.data(), dl);
    std::vector<uint16_t> out(M * K, 0);
    if (or_decode(stored.data(), stored.size(), a.bases.data(), a.hdr.data(), lut_a.data(), a.low.data(), M, K, elem,
                  out.data(), 0) != 0)
        return fail("decode call", M, K, elem);
    if (out != expect) return fail("round trip", M, K, elem);
    return 0;
}

}  // namespace

int main() {
    struct Bf16Case { uint64_t M; uint32_t K; double sigma; };
    const Bf16Case bf16_cases[] = {{8, 512, 0.02}, {13, 40, 0.02}, {3, 4097, 0.02}, {100, 1000, 1.0}, {64, 2048, 0.02},
                                   {17, 520, 0.02}, {1, 1, 0.02}, {300, 3000, 0.02}, {1024, 4096, 0.02}};
    const uint64_t fp8_cases[][2] = {{8, 512}, {13, 40}, {3, 4097}, {101, 1000}, {1024, 4096}};
    int cases = 0, bad = 0;
    Rng g{0x9E3779B97F4A7C15ull};
    for (const auto &c : bf16_cases) {
        std::vector<uint16_t> w(c.M * c.K);
        for (auto &v : w) v = bf16_rne((float)(c.sigma * g.normal()));
        for (int layout = 0; layout <= 2; layout++, cases++) bad |= check(w.data(), w, c.M, c.K, layout << 4);
    }
    {                                                         // signs random, magnitudes 2^U(-40, 40): many escapes
        const uint64_t M = 40;
        const uint32_t K = 1000;
        std::vector<uint16_t> w(M * K);
        for (auto &v : w) v = bf16_rne((float)((g.uniform() < 0.5 ? -1.0 : 1.0) * std::exp2(g.uniform() * 80 - 40)));
        for (int layout = 0; layout <= 1; layout++, cases++) bad |= check(w.data(), w, M, K, layout << 4);
    }
    for (const auto &c : fp8_cases) {
        const uint64_t M = c[0];
        const uint32_t K = (uint32_t)c[1];
        std::vector<uint8_t> w(M * K);
        std::vector<uint16_t> expect(M * K);
        for (uint64_t i = 0; i < M * K; i++) {               // quantized N(0, 1) rows scaled into the e4m3 range
            w[i] = or_f32_to_e4m3((float)(60.0 * g.normal()));
            expect[i] = bf16_of_e4m3(w[i]);
        }
        for (int layout = 0; layout <= 2; layout++, cases++) bad |= check(w.data(), expect, M, K, 1 | layout << 4);
    }
    {                                                         // a NaN code is refused before anything is written
        std::vector<uint8_t> w(8 * 512, 0x38);
        w[777] = 0x7F;
        uint64_t info[4];
        nwc_layout(8, 512, 1, info);
        const Encoded a = run_encoder(nwc_encode, w.data(), 8, 512, 1, info);
        if (a.dl != -2) bad |= fail("NaN refusal", 8, 512, 1);
        cases++;
    }
    if (bad) return 1;
    std::printf("selftest: %d cases ok\n", cases);
    return 0;
}
