// kern_gemm.hip -- the prefill product of a dequantized matrix: Y[T x N] = X[T x K] W[N x K]^T (+ bias), BF16 in and
// out, fp32 accumulation on the matrix cores (v_mfma_f32_16x16x32_bf16).  The reference's prefill multiplies the
// dequantized matrix with cuBLAS (nwc/nwc_torch.py:320-323).  When the output has few 128 x 128 tiles against the
// CUs (2560 rows x 512 tokens: 80 tiles on 256 CUs), K is split over up to 16 workgroups per tile, and the last
// workgroup of a tile to finish adds the partial tiles in split order, so the result does not depend on the order in
// which they finish.  The Python side calls it for the shapes where it measured faster than hipBLASLt (a large K at
// a few hundred tokens: the down projection); hipBLASLt stays faster on the others.
#include "nwc_launch.h"

#include <mutex>

namespace nwc {

// Workspace of nwc_gemm_xbf16_noalloc, for callers that cannot allocate: one copy per GPU, held until the process
// ends.  Host code uses the address hipGetSymbolAddress gives for the current device, never this name.
static __device__ __attribute__((aligned(256))) uint8_t scratch[kGemmScratchBytes];

namespace {

constexpr uint32_t kGT = 128;               // tokens per tile
constexpr uint32_t kGN = 128;               // W rows (output features) per tile
constexpr uint32_t kGK = 64;                // columns per stage

typedef __attribute__((ext_vector_type(8))) __bf16 g_bf16x8;
typedef __attribute__((ext_vector_type(4))) float g_f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t g_u32x4;

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;          // NaN stays a (quiet) NaN
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

struct GemmAcc { g_f32x4 v[4][4]; };

// Y = acc (+ bias), RNE to BF16: acc.v[i][j][e] = Y[token tt*128 + 64 wt + 16 j + (lane & 15)][row tn*128 + 64 wn
// + 16 i + 4 (lane >> 4) + e]
__device__ __forceinline__ void gemm_write_y(const GemmArgs &g, const GemmAcc &acc, uint32_t tt, uint32_t tn,
                                             uint32_t wt, uint32_t wn, uint32_t lane) {
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        const uint32_t t = tt * kGT + 64u * wt + 16u * jj + (lane & 15u);
        if (t >= g.T) continue;
        uint16_t *yr = g.y + (size_t)t * g.N;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t n0 = tn * kGN + 64u * wn + 16u * i + 4u * (lane >> 4);
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                v[e] = acc.v[i][jj][e] + (g.bias && n0 + e < g.N ? __uint_as_float((uint32_t)g.bias[n0 + e] << 16) : 0.f);
            if ((g.N & 3u) == 0u && n0 < g.N) {
                *(uint2 *)(yr + n0) = make_uint2(f32_to_bf16_rne(v[0]) | f32_to_bf16_rne(v[1]) << 16,
                                                 f32_to_bf16_rne(v[2]) | f32_to_bf16_rne(v[3]) << 16);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (n0 + e < g.N) yr[n0 + e] = (uint16_t)f32_to_bf16_rne(v[e]);
            }
        }
    }
}

typedef __attribute__((address_space(3))) void g_lds_void;
typedef __attribute__((address_space(1))) const void g_glob_void;

// A workgroup of four waves owns one 128 x 128 tile of Y and one of the S column ranges (whole 64-column stages);
// wave w computes tokens 64 (w & 1) .. +63 x rows 64 (w >> 1) .. +63 as 4 x 4 MFMA tiles of 16 x 16.  The stages
// go straight from global memory into LDS (global_load_lds_dwordx4: lane l of a wave's load lands at the
// instruction's LDS base + 16 l) through a ring of four stage buffers (128 KB), three stages ahead, with no register
// staging and no LDS store instructions.  A buffer row is 64 BF16 (128 bytes) without padding; row r keeps its
// 16-byte chunk c at slot c ^ f(r), f(r) = (r & 7) ^ ((r >> 3) & 1), so the 16 rows an operand load reads at one
// chunk hit 16 different slots.
__global__ __launch_bounds__(256) void k_gemm_xwt(GemmArgs g) {
    // one array per ring slot: [W, X][row][column]
    __shared__ __attribute__((aligned(16))) uint16_t ring0[2][kGT * kGK], ring1[2][kGT * kGK], ring2[2][kGT * kGK],
        ring3[2][kGT * kGK];
    __shared__ uint32_t last;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
    const uint32_t wt = wv & 1u, wn = wv >> 1;
    // Workgroups go to the eight XCDs in turn (id % 8).  Number them so that each XCD holds a contiguous run of
    // logical ids, and let the token tile vary fastest: the tiles that share a W slab then run on one XCD and read
    // it through the same L2.
    const uint32_t G = gridDim.x, id = blockIdx.x, xcd = id & 7u, slot = id >> 3, G8 = G >> 3, rem = G & 7u;
    const uint32_t L = xcd < rem ? xcd * (G8 + 1u) + slot : rem * (G8 + 1u) + (xcd - rem) * G8 + slot;
    const uint32_t tt = L % g.nT, rest = L / g.nT, split = rest % g.S, tn = rest / g.S;
    const uint32_t s0 = split * g.stages / g.S, ns = (split + 1u) * g.stages / g.S - s0;

    // load i of a wave fills rows 32 wv + 8 i .. +7 of an operand: lane l takes row + (l >> 3), slot l & 7, so it
    // fetches chunk (l & 7) ^ f(row) = (l & 7) ^ (l >> 3) ^ (i & 1); rows past T or N repeat the last row
    const g_u32x4 *wp[4], *xp[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t r = 32u * wv + 8u * i + (lane >> 3), chunk = (lane & 7u) ^ (lane >> 3) ^ (uint32_t)(i & 1);
        const uint32_t rn = min(tn * kGN + r, g.N - 1u), rt = min(tt * kGT + r, g.T - 1u);
        wp[i] = (const g_u32x4 *)(g.w + (size_t)rn * g.ldw + (size_t)s0 * kGK + 8u * chunk);
        xp[i] = (const g_u32x4 *)(g.x + (size_t)rt * g.ldx + (size_t)s0 * kGK + 8u * chunk);
    }
    auto issue = [&](uint16_t (*buf)[kGT * kGK], uint32_t s) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_global_load_lds((g_glob_void *)(wp[i] + (size_t)s * (kGK / 8u)),
                                             (g_lds_void *)&buf[0][(32u * wv + 8u * i) * kGK], 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_global_load_lds((g_glob_void *)(xp[i] + (size_t)s * (kGK / 8u)),
                                             (g_lds_void *)&buf[1][(32u * wv + 8u * i) * kGK], 16, 0, 0);
    };
    // operand loads: lane l reads row (l & 15) of a 16-row subtile, chunk k/8 + (l >> 4) of the k-step at column k
    const uint32_t swz = (lane & 7u) ^ ((lane >> 3) & 1u);
    uint32_t fa[2], fb[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        fa[k] = (wn * 64u + (lane & 15u)) * kGK + 8u * ((4u * k + (lane >> 4)) ^ swz);
        fb[k] = (wt * 64u + (lane & 15u)) * kGK + 8u * ((4u * k + (lane >> 4)) ^ swz);
    }
    GemmAcc acc;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc.v[i][j] = g_f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t last_s = ns - 1u;
    // The operand reads are inline ds_read_b128: the compiler would otherwise wait for every direct load in flight
    // (vmcnt(0)) before any LDS read.  Their results pass through the lgkmcnt(0) wait below, so no matrix-core op can
    // use them before they have arrived.
    auto compute = [&](const uint16_t (*buf)[kGT * kGK]) {
        const uint32_t bw = (uint32_t)(uintptr_t)(g_lds_void *)&buf[0][0], bx = (uint32_t)(uintptr_t)(g_lds_void *)&buf[1][0];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            g_u32x4 a0, a1, a2, a3, x0, x1, x2, x3;
            const uint32_t pa = bw + 2u * fa[k], pb = bx + 2u * fb[k];
            asm volatile("ds_read_b128 %0, %1" : "=v"(a0) : "v"(pa));
            asm volatile("ds_read_b128 %0, %1 offset:2048" : "=v"(a1) : "v"(pa));
            asm volatile("ds_read_b128 %0, %1 offset:4096" : "=v"(a2) : "v"(pa));
            asm volatile("ds_read_b128 %0, %1 offset:6144" : "=v"(a3) : "v"(pa));
            asm volatile("ds_read_b128 %0, %1" : "=v"(x0) : "v"(pb));
            asm volatile("ds_read_b128 %0, %1 offset:2048" : "=v"(x1) : "v"(pb));
            asm volatile("ds_read_b128 %0, %1 offset:4096" : "=v"(x2) : "v"(pb));
            asm volatile("ds_read_b128 %0, %1 offset:6144" : "=v"(x3) : "v"(pb));
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3));
            const g_bf16x8 a[4] = {__builtin_bit_cast(g_bf16x8, a0), __builtin_bit_cast(g_bf16x8, a1),
                                   __builtin_bit_cast(g_bf16x8, a2), __builtin_bit_cast(g_bf16x8, a3)};
            const g_bf16x8 x[4] = {__builtin_bit_cast(g_bf16x8, x0), __builtin_bit_cast(g_bf16x8, x1),
                                   __builtin_bit_cast(g_bf16x8, x2), __builtin_bit_cast(g_bf16x8, x3)};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
                    acc.v[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], x[jj], acc.v[i][jj], 0, 0, 0);
        }
    };
    issue(ring0, 0);
    issue(ring1, min(1u, last_s));
    issue(ring2, min(2u, last_s));
    // step J: stage J's eight loads have landed (stages J + 1 and J + 2 may still be in flight); after the barrier
    // every wave's part of it is in LDS and every wave is done with stage J - 1's slot, which takes stage J + 3
#define NWC_GEMM_STEP(J, CUR, NEXT3)                         \
    __builtin_amdgcn_s_waitcnt(0x4F70); /* vmcnt(16) */         \
    __builtin_amdgcn_s_barrier();                               \
    issue(NEXT3, min((J) + 3u, last_s));                        \
    compute(CUR);
    uint32_t j = 0;
    for (; j + 4u <= ns; j += 4u) {
        NWC_GEMM_STEP(j, ring0, ring3)
        NWC_GEMM_STEP(j + 1u, ring1, ring0)
        NWC_GEMM_STEP(j + 2u, ring2, ring1)
        NWC_GEMM_STEP(j + 3u, ring3, ring2)
    }
    if (j < ns) { NWC_GEMM_STEP(j, ring0, ring3) }
    if (j + 1u < ns) { NWC_GEMM_STEP(j + 1u, ring1, ring0) }
    if (j + 2u < ns) { NWC_GEMM_STEP(j + 2u, ring2, ring1) }
#undef NWC_GEMM_STEP
    __builtin_amdgcn_s_waitcnt(0);                   // the clamped loads past the last stage have landed too

    const uint32_t tile = tn * g.nT + tt;
    if (g.S > 1u) {
        // Partial tiles go through agent-scope (sc1) stores and loads, which the L2 of an XCD does not hold back or
        // serve stale; waiting for the stores to complete before the count is raised orders them before it, so
        // the workgroup that raises the count to S reads every partial tile.  No cache-wide write-back or
        // invalidation is needed.
        float *part = g.part + (size_t)tile * g.S * (64u * 256u);
        float *mine = part + (size_t)split * (64u * 256u) + tid;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    __hip_atomic_store(mine + ((i * 4 + jj) * 4 + e) * 256u, acc.v[i][jj][e], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);                 // this thread's stores have completed
        __syncthreads();
        if (tid == 0)
            last = __hip_atomic_fetch_add(&g.cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g.S - 1u;
        __syncthreads();
        if (!last) return;
        // the S partial tiles in split order, each one's 64 loads in flight together
        GemmAcc sum;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int jj = 0; jj < 4; jj++) sum.v[i][jj] = g_f32x4{0.f, 0.f, 0.f, 0.f};
        for (uint32_t q = 0; q < g.S; q++) {
            if (q == split) {
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) sum.v[i][jj] += acc.v[i][jj];
            } else {
                const float *pq = part + (size_t)q * (64u * 256u) + tid;
                GemmAcc v;
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int jj = 0; jj < 4; jj++)
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            v.v[i][jj][e] = __hip_atomic_load(pq + ((i * 4 + jj) * 4 + e) * 256u, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) sum.v[i][jj] += v.v[i][jj];
            }
        }
        acc = sum;
        if (tid == 0) __hip_atomic_store(&g.cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // next launch
    }
    gemm_write_y(g, acc, tt, tn, wt, wn, lane);
}


__global__ void k_gemm_clear_counters(uint32_t *cnt) {
    for (uint32_t i = threadIdx.x; i < kGemmCounters; i += blockDim.x) cnt[i] = 0u;
}

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kScratchDevices];
bool g_scratch_clear[kScratchDevices];     // the counters were cleared by a kernel that ran outside graph capture

}  // namespace

void *gemm_scratch(hipStream_t st, int *err) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kScratchDevices) {
        *err = e != hipSuccess ? (int)e : (int)hipErrorInvalidDevice;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            *err = e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
            return nullptr;
        }
        g_scratch[dev] = p;
    }
    if (!g_scratch_clear[dev]) {
        // The counters start at zero: a kernel clears them (not a memset, which graph capture would record); every
        // product leaves them zero after that.  Under capture the clear becomes part of the graph, so it is
        // repeated until a call outside capture has run it.
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(st, &cap);
        if (e != hipSuccess) {
            *err = (int)e;
            return nullptr;
        }
        hipLaunchKernelGGL(k_gemm_clear_counters, dim3(1), dim3(256), 0, st, (uint32_t *)g_scratch[dev]);
        e = hipGetLastError();
        if (e != hipSuccess) {
            *err = (int)e;
            return nullptr;
        }
        if (cap == hipStreamCaptureStatusNone) g_scratch_clear[dev] = true;
    }
    return g_scratch[dev];
}

uint32_t gemm_splits(uint32_t T, uint32_t N, uint32_t K, int ncu) {
    const uint32_t tiles = ((T + kGT - 1) / kGT) * ((N + kGN - 1) / kGN), units = K / kGK;
    if (tiles >= (uint32_t)ncu * 3u / 4u) return 1u;
    // about one workgroup per CU, at least 8 stages per split, at most 16 splits
    uint32_t s = ((uint32_t)ncu + tiles / 2u) / tiles;
    s = std::min(s, std::max(1u, units / 8u));
    return std::max(1u, std::min(s, 16u));
}

// Workspace of a split product: kGemmCounters tile counters (zero before the first call; every call leaves them zero,
// whatever the shape), then S partial tiles of 64 KB per output tile.
uint64_t gemm_workspace_bytes(uint32_t T, uint32_t N, uint32_t K, int ncu) {
    const uint64_t tiles = (uint64_t)((T + kGT - 1) / kGT) * ((N + kGN - 1) / kGN);
    const uint32_t s = gemm_splits(T, N, K, ncu);
    if (s == 1u) return 0;
    return kGemmCounters * 4u + tiles * s * 64u * 256u * 4u;
}

int launch_gemm_xwt(GemmArgs g, void *ws, int ncu, hipStream_t st) {
    g.nT = (g.T + kGT - 1) / kGT;
    g.stages = g.K / kGK;
    g.S = gemm_splits(g.T, g.N, g.K, ncu);
    const uint32_t tiles = g.nT * ((g.N + kGN - 1) / kGN);
    g.cnt = nullptr;
    g.part = nullptr;
    if (g.S > 1u) {
        if (tiles > kGemmCounters) return -1;
        g.cnt = (uint32_t *)ws;
        g.part = (float *)((uint8_t *)ws + kGemmCounters * 4u);
    }
    hipLaunchKernelGGL(k_gemm_xwt, dim3(tiles * g.S), dim3(256), 0, st, g);
    return (int)hipGetLastError();
}

}  // namespace nwc
