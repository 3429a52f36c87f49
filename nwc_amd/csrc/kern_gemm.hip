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
constexpr uint32_t kGStride = kGK + 8;      // LDS row stride in BF16: 144 bytes, so 16 rows hit 16 distinct bank quads
constexpr uint32_t kGTile = kGT * kGStride;

typedef __attribute__((ext_vector_type(8))) __bf16 g_bf16x8;
typedef __attribute__((ext_vector_type(4))) float g_f32x4;

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;          // NaN stays a (quiet) NaN
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

typedef __attribute__((ext_vector_type(4))) uint32_t g_u32x4;

struct GemmStage { g_u32x4 w[4], x[4]; };
struct GemmAcc { g_f32x4 v[4][4]; };

__device__ __forceinline__ GemmStage gemm_load(const g_u32x4 *const (&wp)[4], const g_u32x4 *const (&xp)[4], uint32_t s) {
    GemmStage r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r.w[i] = wp[i][(size_t)s * (kGK / 8u)];
        r.x[i] = xp[i][(size_t)s * (kGK / 8u)];
    }
    return r;
}

// buf: [W, X][row][column] of one stage; st: the thread's element offset (row tid >> 3, column 8 (tid & 7))
__device__ __forceinline__ void gemm_store(uint16_t (*buf)[kGTile], uint32_t st, const GemmStage &r) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        *(g_u32x4 *)&buf[0][st + 32u * i * kGStride] = r.w[i];
        *(g_u32x4 *)&buf[1][st + 32u * i * kGStride] = r.x[i];
    }
}

__device__ __forceinline__ void gemm_compute(const uint16_t (*buf)[kGTile], uint32_t fa, uint32_t fb, GemmAcc &acc) {
#pragma unroll
    for (uint32_t kk = 0; kk < kGK; kk += 32u) {
        g_bf16x8 a[4], x[4];
#pragma unroll
        for (int i = 0; i < 4; i++) a[i] = *(const g_bf16x8 *)&buf[0][fa + 16u * i * kGStride + kk];
#pragma unroll
        for (int j = 0; j < 4; j++) x[j] = *(const g_bf16x8 *)&buf[1][fb + 16u * j * kGStride + kk];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc.v[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], x[j], acc.v[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_iglp_opt(0);          // let the scheduler interleave the LDS reads with the matrix-core ops
}

// A workgroup owns one 128 x 128 tile of Y and one of the S column ranges.  H groups of four waves each take 1/H of
// the range (H = 2 when the range can be cut into whole 64-column stage pairs): two waves per SIMD, so one wave's
// matrix-core work overlaps the other's LDS and memory waits, and the two halves' sums are added in LDS at the end.
// In a group, wave w computes tokens 64 (w & 1) .. +63 x rows 64 (w >> 1) .. +63 as 4 x 4 MFMA tiles of 16 x 16;
// stages pass through the group's two LDS buffers, each thread holding up to three stages' loads in registers.
template <int H>
__global__ __launch_bounds__(256 * H) void k_gemm_xwt(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[H][2][2][kGTile];     // [group][buffer][W, X][row][column]
    __shared__ uint32_t last;
    const uint32_t tid = threadIdx.x & 255u, h = threadIdx.x >> 8, lane = tid & 63u, wv = tid >> 6;
    const uint32_t wt = wv & 1u, wn = wv >> 1;
    // Workgroups go to the eight XCDs in turn (id % 8).  Number them so that each XCD holds a contiguous run of
    // logical ids, and let the token tile vary fastest: the tiles that share a W slab then run on one XCD and read
    // it through the same L2.
    const uint32_t G = gridDim.x, id = blockIdx.x, xcd = id & 7u, slot = id >> 3, G8 = G >> 3, rem = G & 7u;
    const uint32_t L = xcd < rem ? xcd * (G8 + 1u) + slot : rem * (G8 + 1u) + (xcd - rem) * G8 + slot;
    const uint32_t tt = L % g.nT, rest = L / g.nT, split = rest % g.S, tn = rest / g.S;
    // the split's units of H stages; group h takes stages s0 .. s0 + ns - 1 (every group the same count)
    const uint32_t units = g.stages / H, u0 = split * units / g.S, ns = (split + 1u) * units / g.S - u0;
    const uint32_t s0 = H * u0 + h * ns;

    // global -> LDS: thread tid moves 16 bytes of rows (tid >> 3) + 32 i, columns 8 (tid & 7) .. +7 of each operand;
    // rows past T or N repeat the last row (their products are never stored)
    const uint32_t lr = tid >> 3, lc = (tid & 7u) * 8u;
    const g_u32x4 *wp[4], *xp[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t rn = min(tn * kGN + lr + 32u * i, g.N - 1u), rt = min(tt * kGT + lr + 32u * i, g.T - 1u);
        wp[i] = (const g_u32x4 *)(g.w + (size_t)rn * g.ldw + (size_t)s0 * kGK + lc);
        xp[i] = (const g_u32x4 *)(g.x + (size_t)rt * g.ldx + (size_t)s0 * kGK + lc);
    }
    // MFMA operands: A = 16 W rows x 32 columns, B = 16 tokens x the same 32 columns; lane l holds row (l & 15),
    // columns 8 (l >> 4) .. +7 of each
    const uint32_t fa = (wn * 64u + (lane & 15u)) * kGStride + 8u * (lane >> 4);
    const uint32_t fb = (wt * 64u + (lane & 15u)) * kGStride + 8u * (lane >> 4);
    const uint32_t st = lr * kGStride + lc;
    uint16_t (*const buf)[2][kGTile] = lds[h];
    GemmAcc acc;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc.v[i][j] = g_f32x4{0.f, 0.f, 0.f, 0.f};

    // Stage s0 + j sits in LDS buffer j & 1 and arrives through register set j % 4: the loads run three stages
    // ahead (past the last stage clamped to it, so the sets are assigned unconditionally and never copied).
    const uint32_t last_s = ns - 1u;
    GemmStage r0 = gemm_load(wp, xp, 0), r1 = gemm_load(wp, xp, min(1u, last_s)),
              r2 = gemm_load(wp, xp, min(2u, last_s)), r3;
    gemm_store(buf[0], st, r0);
    __syncthreads();
    // step J: stage J + 3 into its set, stage J from LDS through the matrix cores, stage J + 1 into the other LDS
    // buffer (its last readers, step J - 1, ended at the barrier)
#define NWC_GEMM_STEP(J, RL, RS)                                \
    RL = gemm_load(wp, xp, min((J) + 3u, last_s));              \
    gemm_compute(buf[(J) & 1u], fa, fb, acc);                   \
    gemm_store(buf[((J) + 1u) & 1u], st, RS);                   \
    __syncthreads();
    uint32_t j = 0;
    for (; j + 4u <= ns; j += 4u) {
        NWC_GEMM_STEP(j, r3, r1)
        NWC_GEMM_STEP(j + 1u, r0, r2)
        NWC_GEMM_STEP(j + 2u, r1, r3)
        NWC_GEMM_STEP(j + 3u, r2, r0)
    }
#undef NWC_GEMM_STEP
    // the last 0-3 stages: stage j is in buffer 0, stages j + 1 and j + 2 in r1 and r2
    const uint32_t tail = ns - j;
    if (tail >= 1u) gemm_compute(buf[0], fa, fb, acc);
    if (tail >= 2u) {
        gemm_store(buf[1], st, r1);
        __syncthreads();
        gemm_compute(buf[1], fa, fb, acc);
    }
    if (tail >= 3u) {
        gemm_store(buf[0], st, r2);            // every wave has finished with buffer 0: barrier above
        __syncthreads();
        gemm_compute(buf[0], fa, fb, acc);
    }

    // acc.v[i][j][e] = Y[token tt*128 + 64 wt + 16 j + (lane & 15)][row tn*128 + 64 wn + 16 i + 4 (lane >> 4) + e]
    if constexpr (H == 2) {
        // group 1's sums into LDS (64 KB, 64 floats per thread), group 0 adds them to its own: columns of the first
        // half first, in every launch
        float *red = (float *)&lds[0][0][0][0];
        __syncthreads();                       // every wave is done with the stage buffers
        if (h == 1) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
#pragma unroll
                    for (int e = 0; e < 4; e++) red[((i * 4 + jj) * 4 + e) * 256u + tid] = acc.v[i][jj][e];
        }
        __syncthreads();
        if (h == 0) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc.v[i][jj][e] += red[((i * 4 + jj) * 4 + e) * 256u + tid];
        }
    }
    const uint32_t tile = tn * g.nT + tt;
    if (g.S > 1u) {
        // Partial tiles go through agent-scope (sc1) stores and loads, which the L2 of an XCD does not hold back or
        // serve stale; waiting for the stores to complete before the count is raised orders them before it, so
        // the workgroup that raises the count to S reads every partial tile.  No cache-wide write-back or
        // invalidation is needed.
        float *part = g.part + (size_t)tile * g.S * (64u * 256u);
        if (h == 0) {
            float *mine = part + (size_t)split * (64u * 256u) + tid;
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        __hip_atomic_store(mine + ((i * 4 + jj) * 4 + e) * 256u, acc.v[i][jj][e], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);     // this thread's stores have completed
        }
        __syncthreads();
        if (threadIdx.x == 0)
            last = __hip_atomic_fetch_add(&g.cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g.S - 1u;
        __syncthreads();
        if (!last) return;
        if (h != 0) return;
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
    if (h != 0) return;
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

uint32_t gemm_groups(uint32_t K) { return K % (2u * kGK) == 0 ? 2u : 1u; }

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
    const uint32_t tiles = ((T + kGT - 1) / kGT) * ((N + kGN - 1) / kGN), units = K / kGK / gemm_groups(K);
    if (tiles >= (uint32_t)ncu * 3u / 4u) return 1u;
    // about one workgroup per CU, at least 8 stage units per split, at most 16 splits
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
    if (gemm_groups(g.K) == 2u)
        hipLaunchKernelGGL(k_gemm_xwt<2>, dim3(tiles * g.S), dim3(512), 0, st, g);
    else
        hipLaunchKernelGGL(k_gemm_xwt<1>, dim3(tiles * g.S), dim3(256), 0, st, g);
    return (int)hipGetLastError();
}

}  // namespace nwc
