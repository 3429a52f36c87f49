// abi.cpp -- device entry points of the C ABI (declared in include/nwc_ops.h): argument checks, launch plans and
// dispatch to the kernel files.  Argument meaning and return codes follow parda21/NWC csrc/nwc_ops.cu:1045-1192.
#include "nwc_launch.h"
#include "nwc_ops.h"

#include <algorithm>
#include <atomic>
#include <cstdlib>

using namespace nwc;

namespace {

constexpr int kMaxDevices = 64;

// NWC_TAIL=0 turns the split-tail layout-0 token plan (k_layout0t) off, for comparisons; read once.
bool tail_enabled() {
    static const bool on = [] {
        const char *v = getenv("NWC_TAIL");
        return !(v && v[0] == '0');
    }();
    return on;
}
std::atomic<int> g_cus[kMaxDevices];

int current_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    int c = g_cus[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) return 0;
    g_cus[dev].store(c, std::memory_order_relaxed);
    return c;
}

// nwc_ops.cu:1050: the fixed block of 4096 weights, M = n / K within 32 bits, and a known element type / layout.
// This build also addresses the raw planes with 32-bit offsets: layout 0 counts weights of the padded matrix
// (Mp * K16, rows past M included), layouts 1/2 count bytes of the plane padded to 16 rows and 32 columns plus its
// 512 slack bytes; both must stay below 2^32.
// Bits 8-15 of elem (a fixed-slot stride, layouts 0/1) are this build's; the reference's callers leave them zero.
bool shape_ok(uint64_t n, uint32_t block, uint32_t K, int elem) {
    if (!(block == kBlock && K != 0 && n % K == 0 && n / K >= 1 && n / K <= 0xFFFFFFFFull && elem_type(elem) <= 1 &&
          elem_layout(elem) <= 2 && (elem & ~0xFFFF) == 0 && elem_stride(elem) <= slot_max(elem_layout(elem))))
        return false;
    const uint64_t M = n / K, K16 = (K + 15u) & ~15u;
    if (M * K16 >= (1ull << 32)) return false;          // also keeps Shape's 32-bit fields (M < 2^28) from wrapping
    const Shape f((uint32_t)M, K, elem_layout(elem));
    if ((uint64_t)f.nb * elem_stride(elem) + 128u >= (1ull << 32)) return false;
    if (elem_layout(elem) == 0) return (uint64_t)f.Mp * f.K16 < (1ull << 32);
    return f.low_bytes(elem) + kRawSlack < (1ull << 32);
}

// LDS words per half-wave for a staged block: an 8 x 512 block of N(0, 0.02^2) BF16 needs ~370 words, real model
// weights (2.85-2.99 code bits per weight) ~405; a 16 x 512 block twice that.  Larger blocks decode from global
// memory instead.
constexpr uint32_t kSlotWords0 = 480, kSlotWords1 = 960;
constexpr uint32_t kDynLdsBudget = 48u * 1024u;       // dynamic LDS per workgroup next to the 16 KB decode table

uint32_t slot_words_for(int layout) { return layout == 0 ? kSlotWords0 : layout == 1 ? kSlotWords1 : 0u; }

// Layout 0: a workgroup owns G whole row groups.  Where a tile of at most 32 blocks makes the grid one residency round
// at two workgroups per CU, that G, with one half-wave (or, with the row index, two or four) per block; otherwise
// tiles of at most 32 blocks over several rounds (PIPE = false: every wave decodes at once).  Only blocks of more than
// 32 column blocks (K beyond 16384) are spread over at most 16 half-waves that each decode several blocks, one round
// at a time, through two region buffers (PIPE = true).
constexpr uint32_t kDynLdsPipe = 62u * 1024u;         // two such workgroups per CU next to their decode tables
// A round buffer of 440 words per block holds the ~350-400 words of N(0, 0.02^2) or real-model BF16 blocks (a round
// that does not fit decodes from global memory), so 32 blocks fit two workgroups per CU.
constexpr uint32_t kSlotWords2 = 440;

// With the 13-bit decode table (32 KB of static LDS instead of 16 KB) two workgroups still share a CU's 160 KB when
// their dynamic LDS stays under this; the single-round tiers are tried with it first.
constexpr uint32_t kDynLds13 = 47u * 1024u;

// Planning stages, tried in this order for each decode table: one residency round, then several rounds of tiles of at
// most 32 blocks, then (12-bit table only) the two-buffer kernel.  Every one-round plan, with either table, comes
// before any multi-round plan.
enum Stage { kOneRound, kRounds, kRoundsOrPipe };
bool plan_layout0_tiers(const Shape &f, int mode, int ncu, bool index, uint32_t budget, Stage stage, LaunchPlan &p);
// Layout-0 token path and dequantization with the row index and the 13-bit table, for matrices of one to two row
// groups per CU (k_layout0t): one whole row group on each CU, the finest split of its blocks whose half-waves fit 32,
// and the rest of the row groups cut into TS = 4 quarters (or 2 halves) of their rows, one workgroup each, so that
// every CU decodes about the same rows: Qwen3-4B down (320 row groups: 256 whole + 256 quarters instead of two whole
// groups on 64 CUs; token 13.8 -> 11.2 us, dequantization 26.2 -> 21.2 us) and o_proj (the same count; 11.7 -> 10.7
// us dequantized).  Both kinds of workgroup share one launch shape: one half-wave per block and part.
bool plan_layout0_tail(const Shape &f, int ncu, LaunchPlan &p) {
    const uint32_t groups = f.groups(), CB = f.CB, n = (uint32_t)ncu;
    if (groups <= n || CB > 32u) return false;
    const uint32_t rest = groups - n;
    const uint32_t ts = 4u * rest <= n ? 4u : 2u * rest <= n ? 2u : 0u;
    if (ts == 0u || n > 65535u) return false;
    const uint32_t split = 4u * CB <= 32u ? 4u : 2u * CB <= 32u ? 2u : 1u;
    const uint32_t halves = (split * CB + 1u) & ~1u;
    const uint32_t lds = CB * kSlotWords0 * 4u + kRows0 * CB * 4u;
    if (lds > kDynLds13) return false;
    p = LaunchPlan{};
    p.layout = 0;
    p.seq13 = true;
    p.tail = ts;
    p.split = split;
    p.G = n;                                            // whole row groups (workgroups 0 .. n - 1)
    p.threads = 32u * halves;
    p.grid = n + ts * rest;
    p.slot_words = kSlotWords0;
    p.lds = lds;
    return true;
}

bool plan_layout0(const Shape &f, int mode, int ncu, bool index, bool seq, LaunchPlan &p) {
    const bool t13 = seq && (mode == kToken || mode == kDequant);
    if ((mode == kToken || mode == kDequant) && index && t13 && tail_enabled() && plan_layout0_tail(f, ncu, p))
        return true;
    if (t13 && plan_layout0_tiers(f, mode, ncu, index, kDynLds13, kOneRound, p)) {
        p.seq13 = true;
        return true;
    }
    if (plan_layout0_tiers(f, mode, ncu, index, kDynLdsPipe, kOneRound, p)) return true;
    if (t13 && plan_layout0_tiers(f, mode, ncu, index, kDynLds13, kRounds, p)) {
        p.seq13 = true;
        return true;
    }
    return plan_layout0_tiers(f, mode, ncu, index, kDynLdsPipe, kRoundsOrPipe, p);
}

bool plan_layout0_tiers(const Shape &f, int mode, int ncu, bool index, uint32_t budget, Stage stage, LaunchPlan &p) {
    p = LaunchPlan{};
    p.layout = 0;
    const bool rows = mode == kToken || mode == kF32;
    const uint32_t CB = f.CB, groups = f.groups(), ncu_ = (uint32_t)ncu;
    const uint32_t part = rows ? kRows0 * CB * 4u : 0u;                // row-sum bytes per row group
    auto ceil_div = [](uint32_t a, uint32_t b) { return (a + b - 1u) / b; };
    auto set = [&](bool pipe, uint32_t split, uint32_t G, uint32_t halves, uint32_t slot, uint32_t lds) {
        p.pipe = pipe;
        p.split = split;
        p.G = G;
        p.threads = 32u * halves;
        p.grid = ceil_div(groups, G);
        p.slot_words = slot;
        p.lds = lds;
        return true;
    };
    // One residency round, wgpc workgroups per CU of G = ceil(groups / (wgpc CUs)) row groups each:
    // 1. with the row index, four or two half-waves per block (rows 0-1 / 2-3 / 4-5 / 6-7 or rows 0-3 / 4-7), up to
    //    32 half-waves (16 waves) per workgroup; two per block only up to 20 half-waves when two workgroups share a CU
    //    (up to 32 in the exception below);
    // 2. else one half-wave per block, up to 32 blocks (the 58-VGPR kernel allows 8 waves per SIMD).
    auto one_round = [&](uint32_t wgpc, uint32_t split2_max) {
        const uint32_t G = std::max(1u, ceil_div(groups, wgpc * ncu_)), blocks = G * CB;
        if (index && (rows || mode == kDequant)) {
            const uint32_t lds = blocks * kSlotWords0 * 4u + G * part;
            if (lds <= budget) {
                if (4u * blocks <= 32u) return set(false, 4u, G, 4u * blocks, kSlotWords0, lds);
                if (2u * blocks <= split2_max) return set(false, 2u, G, 2u * blocks, kSlotWords0, lds);
            }
        }
        const uint32_t halves = (blocks + 1u) & ~1u;
        const uint32_t lds = halves * kSlotWords2 * 4u + G * part;
        return blocks <= 32u && lds <= budget && set(false, 1u, G, halves, kSlotWords2, lds);
    };
    // Workgroups per CU: one, with G1 = ceil(groups / CUs), when no CU then decodes more row groups than the busiest
    // CU of the two-per-CU grid (G2 row groups per workgroup, ceil(groups / G2 / CUs) workgroups on it), or when two
    // would leave a workgroup four blocks or fewer; a single workgroup stages its decode table once for the larger
    // tile.  Qwen3-4B qkv (768 groups: 3 per CU instead of 2 x 2) 9.58 -> 8.88 us, o_proj (320 groups, G1 = 2, two
    // half-waves per block) 8.44 -> 8.11, 9728x2560 (1216 groups: 5 instead of 2 x 3) 13.0 -> 11.2, Qwen3-0.6B qkv
    // 4096x1024 and gate_up 6144x1024 11-12% faster.  Otherwise, or when that tile does not fit, two per CU.
    const uint32_t G2 = std::max(1u, ceil_div(groups, 2u * ncu_)), G1 = ceil_div(groups, ncu_);
    const uint32_t load2 = G2 * ceil_div(ceil_div(groups, G2), ncu_);
    // With the row index, a token tile too large to split over two half-waves per block at one workgroup per CU (more
    // than 16 blocks) loses to the two-per-CU tile that can (up to 32 half-waves): 9728x2560 (1216 groups) 256 x
    // (5 groups, 26 half-waves) 11.0-11.3 us -> 406 x (3, 30) 10.9-11.0 us.
    if (stage == kOneRound && index && rows && 2u * G1 * CB > 32u && 2u * G2 * CB <= 32u && one_round(2u, 32u)) return true;
    if (stage == kOneRound) return ((G2 * CB <= 4u || G1 <= load2) && one_round(1u, 32u)) || one_round(2u, 20u);
    // 2m. one block per half-wave over several residency rounds, when one round's tile would exceed 32 blocks: the
    //     largest tile of at most 32 blocks whose LDS fits the budget (24 blocks next to the 13-bit table, 32 next to
    //     the 12-bit one).  The rounds overlap one workgroup's stream copy with another's decode, which the pipelined
    //     tier does inside one workgroup less well: 151936x2560 132.6 -> 104.6 us, 24576x4096 35.3 -> 27.8,
    //     37888x3584 50.8 -> 40.7, 151936x4096 200.5 -> 152.9, 152064x3584 174.5 -> 143.8 (13-bit table).
    if (CB <= 32u) {
        for (uint32_t G = std::min(groups, 32u / CB); G >= 1u; G--) {
            const uint32_t blocks = G * CB, halves = (blocks + 1u) & ~1u;
            const uint32_t lds = halves * kSlotWords0 * 4u + G * part;
            if (lds <= budget) return set(false, 1u, G, halves, kSlotWords0, lds);
        }
    }
    if (stage != kRoundsOrPipe) return false;
    // 3. several blocks per half-wave: rounds through two region buffers, two workgroups per CU
    uint32_t G = std::max(1u, ceil_div(groups, 2u * ncu_));
    for (;; G--) {
        const uint32_t blocks = G * CB;
        uint32_t halves, lds;
        if (blocks <= 20) {
            halves = (blocks + 1u) & ~1u;
            lds = halves * kSlotWords0 * 4u + G * part;
            if (lds <= kDynLdsPipe) return set(false, 1u, G, halves, kSlotWords0, lds);
        } else {
            const uint32_t rounds = (blocks + 15u) / 16u;
            halves = ((blocks + rounds - 1u) / rounds + 1u) & ~1u;
            while (halves > 2 && halves * 2u * kSlotWords0 * 4u + G * part > kDynLdsPipe) halves -= 2;
            lds = halves * 2u * kSlotWords0 * 4u + G * part;
            if (lds <= kDynLdsPipe) return set(true, 1u, G, halves, kSlotWords0, lds);
        }
        if (G == 1) return false;                            // K beyond ~190k columns
    }
}

// Layout-0 token path for ntok activation vectors at once (k_layout0_batch): one half-wave per block, ntok partial
// sums per row.  The one-round tile of the two-per-CU grid when it is small enough, else the largest such tile over
// several rounds; at each stage the 13-bit table first (with `seq`), then the 12-bit LUT.
bool plan_layout0_batch(const Shape &f, int ncu, uint32_t ntok, bool seq, LaunchPlan &p) {
    const uint32_t CB = f.CB, groups = f.groups(), part = kRows0 * CB * 4u * ntok;
    // blocks per tile (at least one row group's): the kernel takes 62-67 VGPRs for two vectors (7-8 waves per SIMD),
    // 71-75 for three (6), 87-88 for four (5), so larger batches want smaller tiles; swept on MI355X (gate_up
    // 19456x2560: three vectors 22.0 us at 20 blocks against 23.5-25.6 at 12-32, four 25.3 us at 15-16 against
    // 30.2 at 20 and 27.0 at 25-32; qkv flat; down takes its whole 19-block row group)
    if (CB > 32u) return false;
    const uint32_t cap = std::max(CB, ntok <= 2u ? 32u : ntok == 3u ? 20u : 16u);
    auto fit = [&](uint32_t G, uint32_t budget, uint32_t slot) {
        const uint32_t blocks = G * CB, halves = (blocks + 1u) & ~1u, lds = halves * slot * 4u + G * part;
        if (blocks > cap || lds > budget) return false;
        p = LaunchPlan{};
        p.layout = 0;
        p.split = 1;
        p.seq13 = budget == kDynLds13;
        p.G = G;
        p.threads = 32u * halves;
        p.grid = (groups + G - 1u) / G;
        p.slot_words = slot;
        p.lds = lds;
        return true;
    };
    const uint32_t G2 = std::max(1u, (groups + 2u * (uint32_t)ncu - 1u) / (2u * (uint32_t)ncu));
    for (uint32_t budget : {kDynLds13, kDynLdsPipe})
        if ((seq || budget != kDynLds13) && fit(G2, budget, kSlotWords2)) return true;
    for (uint32_t budget : {kDynLds13, kDynLdsPipe}) {
        if (!seq && budget == kDynLds13) continue;
        for (uint32_t G = std::min(G2, cap / CB); G >= 1u; G--)
            if (fit(G, budget, kSlotWords0)) return true;
    }
    return false;
}

// Layout 1, single round, for the token path and dequantization with the row index: G whole 16-row groups per
// workgroup (two workgroups per CU), SP = 4 or 2 half-waves per block, at most 32 half-waves; a region buffer of up to
// 880 words per block (a 16 x 512 block of N(0, 0.02^2) BF16 needs ~700, real model weights ~760).  Building the index
// itself uses SP = 1 (decoding from global memory: the region is larger than the copy's four chunks per thread), and
// so does dequantization without the index (its copy finishes the region in a second pass).  False otherwise: the
// caller then uses the multi-block kernel.
constexpr uint32_t kSlotWords1s = 880, kSlotWords1Min = 768;
constexpr uint32_t kDynLdsOne = 128u * 1024u;         // dynamic LDS of a workgroup that has its CU to itself
constexpr uint32_t kDynLdsOne13 = 126u * 1024u;       // the same next to the 13-bit table
bool plan_layout1_budget(const Shape &f, int mode, int ncu, bool index, uint32_t budget, uint32_t one, Stage stage,
                         LaunchPlan &p);
// Dequantization of a layout-1 matrix in one round: tiles of whole blocks instead of whole row groups (G = blocks |
// 1 << 31), two per CU, so every CU decodes about the same number of blocks (there are no row sums to combine):
// 2560 x 9728 has 160 row groups of 19 blocks for 256 CUs, 507 tiles of 6 blocks; 19456 x 2560 1216 row groups of 5,
// 507 tiles of 12 (whole row groups: 406 tiles of 3, so some CUs decode 6 row groups and others 3).  Four (or two)
// half-waves per block, which needs the row index, at most 32 per workgroup; the 13-bit table when given.  Larger
// matrices keep the row-group plans.
bool plan_layout1_blocks(const Shape &f, int ncu, bool seq, LaunchPlan &p) {
    const uint32_t nb = f.nb, n = 2u * (uint32_t)ncu, BT = std::max(1u, (nb + n - 1u) / n);
    if (BT > 16u) return false;
    for (int pass = 0; pass < 2; pass++) {
        const bool t13 = pass == 0;
        if (t13 && !seq) continue;
        const uint32_t budget = t13 ? kDynLds13 : kDynLdsPipe;
        if (BT * kSlotWords1Min * 4u > budget) continue;
        for (uint32_t sp : {4u, 2u}) {
            const uint32_t halves = (BT * sp + 1u) & ~1u;
            if (halves > 32u) continue;
            const uint32_t slot = std::min(kSlotWords1s, budget / (4u * BT));
            p = LaunchPlan{};
            p.layout = 1;
            p.seq13 = t13;
            p.split = sp;
            p.G = BT | 0x80000000u;
            p.threads = 32u * halves;
            p.grid = (nb + BT - 1u) / BT;
            p.slot_words = slot;
            p.lds = BT * slot * 4u;
            return true;
        }
    }
    return false;
}

bool plan_layout1(const Shape &f, int mode, int ncu, bool index, bool seq, LaunchPlan &p) {
    if (mode == kDequant && index && plan_layout1_blocks(f, ncu, seq, p)) return true;
    const bool t13 = seq && ((mode == kToken && index) || mode == kDequant);
    for (Stage stage : {kOneRound, kRounds}) {
        if (t13 && plan_layout1_budget(f, mode, ncu, index, kDynLds13, kDynLdsOne13, stage, p)) {
            p.seq13 = true;
            return true;
        }
        if (plan_layout1_budget(f, mode, ncu, index, kDynLdsPipe, kDynLdsOne, stage, p)) return true;
    }
    return false;
}
bool plan_layout1_budget(const Shape &f, int mode, int ncu, bool index, uint32_t budget, uint32_t one, Stage stage,
                         LaunchPlan &p) {
    p = LaunchPlan{};
    p.layout = 1;
    const bool rows = mode == kToken || mode == kF32;
    const uint32_t CB = f.CB, groups = f.groups();
    auto tile = [&](uint32_t G) {
        const uint32_t blocks = G * CB;
        for (uint32_t sp : {4u, 2u, 1u}) {
            if (sp > 1 ? !(index && (rows || mode == kDequant)) : (mode != kRowIndex && mode != kDequant)) continue;
            const uint32_t halves = (blocks * sp + 1u) & ~1u;
            if (halves > 32u) continue;
            const uint32_t part = rows ? G * kRows12 * CB * sp * 4u + (f.K16 + 31u) / 32u * 64u : 0u;   // + x as BF16
            if (part + blocks * kSlotWords1Min * 4u > budget) continue;
            const uint32_t slot = std::min(kSlotWords1s, (budget - part) / (4u * blocks));
            p.split = sp;
            p.G = G;
            p.threads = 32u * halves;
            p.grid = (groups + G - 1u) / G;
            p.slot_words = slot;
            p.lds = blocks * slot * 4u + part;
            return true;
        }
        return false;
    };
    const uint32_t G1 = std::max(1u, (groups + 2u * (uint32_t)ncu - 1u) / (2u * (uint32_t)ncu));
    if (stage == kRounds) {
        // several residency rounds (the vocabulary matrices: 151936x2560 has 9496 groups): the largest tile that
        // fits (151936x2560 token path, the row index now built as well: BF16 197.6 -> 113.5 us, fp8 237.1 -> 104.4)
        for (uint32_t G = std::min(G1 - 1u, 32u / CB); G >= 1u; G--)
            if (tile(G)) return true;
        return false;
    }
    if (tile(G1)) return true;
    // several items per half-wave: one 16-row group per workgroup, 32 half-waves, up to kDynLdsOne of LDS (one such
    // workgroup per CU; the region copy moves at most 64 KB)
    if (index && mode == kToken && CB * 4u > 32u) {
        const uint32_t part = kRows12 * CB * 4u * 4u + (f.K16 + 31u) / 32u * 64u;
        const uint32_t slot = std::min(kSlotWords1s, (one - part) / (4u * CB));
        if (slot >= kSlotWords1Min && CB * kSlotWords1Min * 4u <= 64u * 1024u) {
            p.split = 4;
            p.multi = true;
            p.G = 1;
            p.threads = 1024;
            p.grid = groups;
            p.slot_words = slot;
            p.lds = CB * slot * 4u + part;
            return true;
        }
    }
    return false;
}

// Layouts 1/2: workgroup tile = G whole row groups, one block per half-wave where the LDS budget allows.  Prefer at
// least two workgroups per CU (small matrices spread over the whole chip), at most 32 blocks (16 waves) per
// workgroup, and an even block count so both halves of every wave have a block.
bool plan_blocks(const Shape &f, int layout, int mode, int ncu, bool index, LaunchPlan &p, bool seq = false,
                 bool fp8 = false) {
    if (layout == 0) return plan_layout0(f, mode, ncu, index, seq, p);
    if (layout == 1 && plan_layout1(f, mode, ncu, index, seq, p)) return true;
    if (mode == kRowIndex) return false;
    p = LaunchPlan{};
    p.layout = layout;
    const uint32_t CB = f.CB, groups = f.groups(), slot = slot_words_for(layout);
    // layout 2, BF16 token path: G = ceil(groups / (2 CUs)) whole row groups per workgroup, each block's 16
    // super-chunks split into four (or two) ranges.  With at most 32 ranges per tile, one half-wave each (7B qkv, o);
    // otherwise four ranges per block go round-robin over 32 half-waves (7B gate_up: 41.2 -> 36.5-36.9 us against one
    // half-wave per block, down 25.9 -> 23.7).  x is staged in LDS as BF16 (the token path of layouts 1/2 always
    // takes BF16 x).
    if (layout == 2 && !fp8 && mode == kToken) {
        const uint32_t G = std::max(1u, (groups + 2u * (uint32_t)ncu - 1u) / (2u * (uint32_t)ncu));
        auto lds_sp = [&](uint32_t sp) { return (f.K16 + 31u) / 32u * 64u + G * f.rows * CB * sp * 4u; };
        auto take = [&](uint32_t sp, uint32_t halves) {
            p.split = sp;
            p.G = G;
            p.threads = 32u * halves;
            p.grid = (groups + G - 1u) / G;
            p.lds = lds_sp(sp);
            return true;
        };
        for (uint32_t sp : {4u, 2u}) {
            const uint32_t halves = (G * CB * sp + 1u) & ~1u;
            if (halves <= 32u && lds_sp(sp) <= kDynLdsPipe) return take(sp, halves);
        }
        if (lds_sp(4u) <= kDynLdsPipe) return take(4u, 32u);
    }
    uint32_t G = CB >= 32 ? 1u : 32u / CB;
    while (G > 1 && (groups + G - 1) / G < 2u * (uint32_t)ncu) G--;
    if (G > 1 && ((G * CB) & 1u)) G--;
    // layout 2's token path when the split's partial sums do not fit (whole blocks, one round): at most two
    // workgroups per CU even if a tile then holds more blocks than half-waves
    if (layout == 2 && !fp8 && mode == kToken && CB < 32u)
        G = std::max(G, (groups + 2u * (uint32_t)ncu - 1u) / (2u * (uint32_t)ncu));
    if (G > groups) G = groups;
    if (G == 0) G = 1;
    auto lds_of = [&](uint32_t g, uint32_t halves) {
        return halves * slot * 4u + (mode == kDequant ? 0u : g * f.rows * CB * 4u);
    };
    uint32_t halves = std::min(32u, (G * CB + 1) & ~1u);
    while (G > 1 && lds_of(G, halves) > kDynLdsBudget) {
        G--;
        halves = std::min(32u, (G * CB + 1) & ~1u);
    }
    while (halves > 2 && lds_of(G, halves) > kDynLdsBudget) halves -= 2;   // several blocks per half-wave
    if (lds_of(G, halves) > kDynLdsBudget) return false;                     // K beyond ~190k columns
    p.G = G;
    p.threads = 32u * halves;
    p.grid = (groups + G - 1) / G;
    p.lds = lds_of(G, halves);
    if (layout == 2 && !fp8 && mode == kToken) {        // the single-round kernel with one half-wave per block
        // (activations staged in LDS and loads four super-chunks ahead: 7B gate_up 47.6 -> 43.6 us, down 27.6 -> 25.9)
        const uint32_t xb = (f.K16 + 31u) / 32u * 64u;
        if (p.lds + xb <= kDynLdsPipe) {
            p.split = 1;
            p.lds += xb;
        }
    }
    return true;
}

int run_blocks(int mode, bool xbf16, hipStream_t st, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr,
               const uint32_t *tab, const uint8_t *low, const void *x, const uint16_t *bias, const float *scale, void *out,
               uint64_t n, uint32_t K, int elem, const uint16_t *aux = nullptr, const uint32_t *seq = nullptr) {
    const int ncu = current_cus();
    if (ncu <= 0) return (int)hipErrorNoDevice;
    const int layout = elem_layout(elem), t = elem_type(elem);
    const Shape f((uint32_t)(n / K), K, layout);
    LaunchPlan p;
    if (!plan_blocks(f, layout, mode, ncu, aux != nullptr && layout <= 1, p, seq != nullptr && layout <= 1 && xbf16,
                     t == kElemFp8))
        return -1;
    BlockArgs a{data, bases, hdr, tab, low, x, bias, scale, out, aux, f.M, f.K, p.G,
                layout == 0 || p.split ? p.slot_words : slot_words_for(layout), seq, elem_stride(elem)};
    return layout == 2 ? launch_fixed(p, t, mode, xbf16, a, st) : launch_prefix(p, t, mode, xbf16, a, st);
}

}  // namespace

extern "C" int nwc_ref_bf16(void *stream, const uint16_t *w, const uint16_t *x, uint16_t *y, uint64_t M, uint32_t K) {
    if (M == 0 || K == 0 || M > 0xFFFFFFFFull) return -1;
    const int ncu = current_cus();
    if (ncu <= 0) return (int)hipErrorNoDevice;
    return launch_ref_bf16(w, x, y, (uint32_t)M, K, ncu, (hipStream_t)stream);
}

extern "C" uint64_t nwc_gemm_workspace(uint32_t T, uint32_t N, uint32_t K) {
    const int ncu = current_cus();
    return ncu > 0 ? gemm_workspace_bytes(T, N, K, ncu) : 0;
}

namespace {
bool gemm_args_ok(const uint16_t *x, uint32_t ldx, const uint16_t *w, uint32_t ldw, const uint16_t *bias,
                  const uint16_t *y, uint32_t T, uint32_t N, uint32_t K) {
    return !(T == 0 || N == 0 || K == 0 || K % 64u != 0 || ldx < K || ldw < K || ldx % 8u != 0 || ldw % 8u != 0 ||
             ((uintptr_t)x & 15u) != 0 || ((uintptr_t)w & 15u) != 0 || ((uintptr_t)y & 7u) != 0 ||
             ((uintptr_t)bias & 1u) != 0 || (uint64_t)T * N >= (1ull << 32));
}
}  // namespace

extern "C" int nwc_gemm_xbf16(void *stream, const uint16_t *x, uint32_t ldx, const uint16_t *w, uint32_t ldw,
                              const uint16_t *bias, uint16_t *y, uint32_t T, uint32_t N, uint32_t K, void *ws,
                              uint64_t ws_bytes) {
    if (!gemm_args_ok(x, ldx, w, ldw, bias, y, T, N, K)) return -1;
    const int ncu = current_cus();
    if (ncu <= 0) return (int)hipErrorNoDevice;
    const uint64_t need = gemm_workspace_bytes(T, N, K, ncu);
    if (need && (ws == nullptr || ws_bytes < need || ((uintptr_t)ws & 255u) != 0)) return -1;
    GemmArgs g{x, w, bias, y, nullptr, nullptr, ldx, ldw, T, N, K, 0, 0, 0};
    return launch_gemm_xwt(g, ws, ncu, (hipStream_t)stream);
}

extern "C" int nwc_gemm_xbf16_noalloc(void *stream, const uint16_t *x, uint32_t ldx, const uint16_t *w, uint32_t ldw,
                                      const uint16_t *bias, uint16_t *y, uint32_t T, uint32_t N, uint32_t K) {
    if (!gemm_args_ok(x, ldx, w, ldw, bias, y, T, N, K)) return -1;
    const int ncu = current_cus();
    if (ncu <= 0) return (int)hipErrorNoDevice;
    const uint64_t need = gemm_workspace_bytes(T, N, K, ncu);
    if (need > kGemmScratchBytes) return -1;
    void *ws = nullptr;
    if (need) {
        int err = 0;
        ws = gemm_scratch((hipStream_t)stream, &err);
        if (ws == nullptr) return err ? err : (int)hipErrorInvalidValue;
    }
    GemmArgs g{x, w, bias, y, nullptr, nullptr, ldx, ldw, T, N, K, 0, 0, 0};
    return launch_gemm_xwt(g, ws, ncu, (hipStream_t)stream);
}

extern "C" int nwc_stream_read(void *stream, const void *p, uint64_t bytes, uint32_t *out, uint32_t grid) {
    if (bytes == 0 || bytes % 16 != 0 || ((uintptr_t)p & 15u) != 0 || grid == 0) return -1;
    if (current_cus() <= 0) return (int)hipErrorNoDevice;
    return launch_stream_read(p, bytes, out, grid, (hipStream_t)stream);
}

extern "C" int nwc_setup(void) { return current_cus(); }

extern "C" int nwc_matvec(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                          const uint8_t *low, const float *x, float *y, uint64_t n, uint32_t block, uint32_t K, int elem) {
    if (!shape_ok(n, block, K, elem)) return -1;
    return run_blocks(kF32, false, (hipStream_t)stream, data, bases, hdr, tab, low, x, nullptr, nullptr, y, n, K, elem);
}

extern "C" int nwc_dequant(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                           const uint8_t *low, uint16_t *out, uint64_t n, uint32_t block, uint32_t K, int elem) {
    if (!shape_ok(n, block, K, elem)) return -1;
    return run_blocks(kDequant, true, (hipStream_t)stream, data, bases, hdr, tab, low, nullptr, nullptr, nullptr, out, n, K, elem);
}

extern "C" int nwc_dequant_seq(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr,
                               const uint32_t *tab, const uint8_t *low, const uint16_t *row_index,
                               const uint32_t *seq_table, uint16_t *out, uint64_t n, uint32_t K, int elem) {
    if (!shape_ok(n, kBlock, K, elem)) return -1;
    const int layout = elem_layout(elem);
    return run_blocks(kDequant, true, (hipStream_t)stream, data, bases, hdr, tab, low, nullptr, nullptr, nullptr, out, n, K,
                      elem, layout <= 1 ? row_index : nullptr, layout <= 1 ? seq_table : nullptr);
}

extern "C" int nwc_linear_bf16(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                               const uint8_t *low, const float *x, const uint16_t *bias, const float *scale, float *scratch,
                               uint16_t *y, uint64_t n, uint32_t block, uint32_t K, int elem) {
    (void)scratch;
    if (!shape_ok(n, block, K, elem)) return -1;
    const bool xbf16 = elem_layout(elem) != 0;                    // layout 0 takes fp32 x, layouts 1/2 BF16 x
    return run_blocks(kToken, xbf16, (hipStream_t)stream, data, bases, hdr, tab, low, x, bias, scale, y, n, K, elem);
}

extern "C" int nwc_linear_xbf16(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                                const uint8_t *low, const uint16_t *row_index, const uint32_t *seq_table, const uint16_t *x,
                                const uint16_t *bias, const float *scale, uint16_t *y, uint64_t n, uint32_t K, int elem) {
    if (!shape_ok(n, kBlock, K, elem)) return -1;
    return run_blocks(kToken, true, (hipStream_t)stream, data, bases, hdr, tab, low, x, bias, scale, y, n, K, elem,
                      elem_layout(elem) <= 1 ? row_index : nullptr, elem_layout(elem) <= 1 ? seq_table : nullptr);
}

extern "C" int nwc_linear_xbf16_batch(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr,
                                      const uint32_t *tab, const uint8_t *low, const uint32_t *seq_table, const uint16_t *x,
                                      const uint16_t *bias, const float *scale, uint16_t *y, uint64_t n, uint32_t K,
                                      int elem, uint32_t ntok) {
    if (!shape_ok(n, kBlock, K, elem) || elem_layout(elem) != 0 || ntok < 1 || ntok > 4) return -1;
    if (ntok == 1)
        return run_blocks(kToken, true, (hipStream_t)stream, data, bases, hdr, tab, low, x, bias, scale, y, n, K, elem,
                          nullptr, seq_table);
    const int ncu = current_cus();
    if (ncu <= 0) return (int)hipErrorNoDevice;
    const Shape f((uint32_t)(n / K), K, 0);
    LaunchPlan p;
    if (!plan_layout0_batch(f, ncu, ntok, seq_table != nullptr, p)) return -1;
    BlockArgs a{data, bases, hdr, tab, low, x, bias, scale, y, nullptr, f.M, f.K, p.G, p.slot_words, seq_table,
                elem_stride(elem)};
    return launch_layout0_batch(p, elem_type(elem), a, ntok, (hipStream_t)stream);
}

// Prefill (ntok >= 1 tokens) of a layout-0 matrix without a temporary BF16 matrix (k_prefill0).  Token tile: the
// largest of 256, 128, 64 that the tokens need and that still gives the 64-row tiles at least one workgroup per CU
// (each token tile decodes the matrix once more).
uint32_t prefill_tokens_per_tile(uint32_t row_tiles, uint32_t ntok, int ncu) {
    uint32_t tt = 256;
    while (tt > 64u && (tt / 2u >= ntok || row_tiles * ((ntok + tt - 1u) / tt) < (uint32_t)ncu)) tt /= 2u;
    return tt;
}

extern "C" int nwc_prefill_xbf16(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr,
                                 const uint32_t *tab, const uint8_t *low, const uint16_t *row_index,
                                 const uint32_t *seq_table, const uint16_t *x, const uint16_t *bias, const float *scale,
                                 uint16_t *y, uint64_t n, uint32_t K, int elem, uint32_t ntok) {
    if (!shape_ok(n, kBlock, K, elem) || elem_layout(elem) != 0 || !row_index || !seq_table) return -1;
    if (ntok == 0) return 0;
    if (ntok > 65535u * 64u) return -1;
    const int ncu = current_cus();
    if (ncu <= 0) return (int)hipErrorNoDevice;
    const Shape f((uint32_t)(n / K), K, 0);
    const uint32_t row_tiles = (f.groups() + 7u) / 8u;
    PrefillArgs p{BlockArgs{data, bases, hdr, tab, low, nullptr, bias, scale, y, row_index, f.M, f.K, 8u, 0u, seq_table,
                            elem_stride(elem)},
                  x, ntok};
    return launch_prefill0(elem_type(elem), prefill_tokens_per_tile(row_tiles, ntok, ncu), p, (hipStream_t)stream);
}

extern "C" int nwc_row_index(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                             const uint8_t *low, uint16_t *row_index, uint64_t n, uint32_t K, int elem) {
    if (!shape_ok(n, kBlock, K, elem) || elem_layout(elem) > 1) return -1;
    return run_blocks(kRowIndex, true, (hipStream_t)stream, data, bases, hdr, tab, low, nullptr, nullptr, nullptr, row_index,
                      n, K, elem);
}

extern "C" int nwc_token_split(uint64_t n, uint32_t K, int elem, int with_row_index) {
    if (!shape_ok(n, kBlock, K, elem)) return -1;
    const int ncu = current_cus();
    if (ncu <= 0) return (int)hipErrorNoDevice;
    const Shape f((uint32_t)(n / K), K, elem_layout(elem));
    LaunchPlan p;
    const bool index = (with_row_index & 1) != 0 && elem_layout(elem) <= 1, seq = (with_row_index & 2) != 0;
    if (!plan_blocks(f, elem_layout(elem), kToken, ncu, index, p, seq && elem_layout(elem) <= 1)) return -1;
    return elem_layout(elem) <= 1 && p.split ? (int)p.split : 1;
}

extern "C" int nwc_gather(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                          const uint8_t *low, const int64_t *ids, uint32_t n_ids, uint16_t *out, uint64_t n, uint32_t block,
                          uint32_t K, int elem) {
    if (!shape_ok(n, block, K, elem)) return -1;
    if (n_ids == 0) return 0;
    if (current_cus() <= 0) return (int)hipErrorNoDevice;
    GatherArgs a{data, bases, hdr, tab, low, ids, n_ids, out, (uint32_t)(n / K), K, slot_words_for(elem_layout(elem))};
    const int layout = elem_layout(elem), t = elem_type(elem);
    return layout == 2 ? launch_gather_fixed(t, a, (hipStream_t)stream) : launch_gather_prefix(layout, t, a, (hipStream_t)stream);
}

extern "C" int nwc_gather_xindex(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr,
                                 const uint32_t *tab, const uint8_t *low, const uint16_t *row_index,
                                 const uint32_t *seq_table, const int64_t *ids, uint32_t n_ids, uint16_t *out, uint64_t n,
                                 uint32_t K, int elem) {
    const int layout = elem_layout(elem);
    if (!shape_ok(n, kBlock, K, elem) || layout > 1 || !row_index) return -1;
    if (n_ids == 0) return 0;
    if (current_cus() <= 0) return (int)hipErrorNoDevice;
    GatherArgs a{data, bases, hdr, tab, low, ids, n_ids, out, (uint32_t)(n / K), K, slot_words_for(layout)};
    return launch_gather0x(layout, elem_type(elem), a, row_index, seq_table, (hipStream_t)stream);
}

extern "C" int nwc_ref_fp8(void *stream, const uint8_t *w, const float *scale, const float *x, uint16_t *y, uint64_t M, uint32_t K) {
    if (M == 0 || K == 0 || M > 0xFFFFFFFFull) return -1;
    const int ncu = current_cus();
    if (ncu <= 0) return (int)hipErrorNoDevice;
    return launch_ref_fp8(w, scale, x, y, (uint32_t)M, K, ncu, (hipStream_t)stream);
}
