// kern_misc.hip -- the uncompressed baselines the compressed path is measured against: the fp8 weight-only matvec
// (the "native fp8" baseline; counterpart of the reference's kern_ref_fp8, nwc_ops.cu:760-829), a BF16 matvec written
// the same way (the uncompressed BF16 bar next to hipBLASLt), and a plain streaming read (the bandwidth a kernel of
// a given size can reach on this GPU).
//
// Bandwidth-tuned: each workgroup streams a few whole rows with every lane keeping several 8-byte loads in flight,
// converts with the gfx950 OCP-e4m3 packed conversion (v_cvt_pk_f32_fp8) and accumulates in fp32 against fp32
// activations; one BF16 store per row.
#include "nwc_device.h"
#include "nwc_launch.h"

#include <algorithm>

namespace nwc {

typedef __attribute__((ext_vector_type(2))) float f32x2_t;

__device__ __forceinline__ float fp8_to_f32_exact(uint32_t b) {
    const uint32_t e = (b >> 3) & 15u, m = b & 7u;
    const float v = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0.001953125f;
    return (b & 0x80u) ? -v : v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Fallback for rows that are not 8-byte aligned (K % 8 != 0) or unaligned pointers: one wave per 4 rows, one byte
// per lane and step, the exact e4m3 value from its fields.
__global__ void __launch_bounds__(256) k_fp8_bytes(const uint8_t *__restrict__ w, const float *__restrict__ scale,
                                                   const float *__restrict__ x, uint16_t *__restrict__ y, uint32_t M, uint32_t K) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 4;
    if (row0 >= M) return;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int r = 0; r < 4; r++) {
        if (row0 + r >= M) break;
        for (uint32_t k = lane; k < K; k += 64) acc[r] = fmaf(fp8_to_f32_exact(w[(uint64_t)(row0 + r) * K + k]), x[k], acc[r]);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float v = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < M) y[row0 + r] = (uint16_t)f32_to_bf16_rne(v * scale[row0 + r]);
    }
}

// Rows of 8-byte-aligned fp8 weights.  A workgroup owns R consecutive rows; its W waves split each row into chunks of
// 512 columns, chunk j going to wave j mod W, so a wave holds at most JB = ceil(J / W) chunks of each row.  Lane l owns
// columns 8l .. 8l + 7 of a chunk: one 8-byte non-temporal load per row (a wave reads 512 contiguous bytes of each of
// its R rows) and two 16-byte loads of x, shared by the R rows.  All of a wave's loads are issued before the first is
// used, x first (it is read by every workgroup, so it comes from L2 and arrives before the weights, which the wait
// counter needs, being in order), so a wave has R x JB x 512 weight bytes in flight at once.  Columns past K and rows
// past M load from in-range addresses and contribute zero.  Partial sums: lane order, then a butterfly over the
// wave, then the W waves in order through LDS; one BF16 store of scale * sum per row.
template <int R, int JB>
__global__ void __launch_bounds__(512) k_fp8_rows(const uint8_t *__restrict__ w, const float *__restrict__ scale,
                                                  const float *__restrict__ x, uint16_t *__restrict__ y, uint32_t M, uint32_t K) {
    __shared__ float part[8][R];
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6, W = blockDim.x >> 6;
    const uint32_t row0 = blockIdx.x * R, J = (K + 511u) >> 9;
    const uint8_t *rp[R];
#pragma unroll
    for (int r = 0; r < R; r++) rp[r] = w + (uint64_t)min(row0 + r, M - 1u) * K;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    for (uint32_t j0 = wv; j0 < J; j0 += W * JB) {
        uint2 q[JB][R];
        float4 xa[JB], xb[JB];
        uint32_t cc[JB];
        bool ok[JB];
#pragma unroll
        for (int b = 0; b < JB; b++) {
            const uint32_t c = (j0 + b * W) * 512u + 8u * lane;
            ok[b] = j0 + b * W < J && c < K;
            cc[b] = ok[b] ? c : 0u;
            if (JB == 1 || j0 + b * W < J) {                      // wave-uniform
                xa[b] = *(const float4 *)(x + cc[b]);
                xb[b] = *(const float4 *)(x + cc[b] + 4);
            }
        }
#pragma unroll
        for (int b = 0; b < JB; b++) {
            if (JB == 1 || j0 + b * W < J) {
#pragma unroll
                for (int r = 0; r < R; r++) q[b][r] = ldnt2(rp[r] + cc[b]);
            }
        }
#pragma unroll
        for (int b = 0; b < JB; b++) {
            if (JB > 1 && j0 + b * W >= J) break;
            const float xv[8] = {xa[b].x, xa[b].y, xa[b].z, xa[b].w, xb[b].x, xb[b].y, xb[b].z, xb[b].w};
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t cw[2] = {ok[b] ? q[b][r].x : 0u, ok[b] ? q[b][r].y : 0u};
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)cw[h], false);
                    const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)cw[h], true);
                    acc[r] = fmaf(lo.x, xv[4 * h], acc[r]);
                    acc[r] = fmaf(lo.y, xv[4 * h + 1], acc[r]);
                    acc[r] = fmaf(hi.x, xv[4 * h + 2], acc[r]);
                    acc[r] = fmaf(hi.y, xv[4 * h + 3], acc[r]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
    if (W == 1) {
        if (lane < (uint32_t)R && row0 + lane < M) {
            float v = acc[0];
#pragma unroll
            for (int r = 1; r < R; r++) v = lane == (uint32_t)r ? acc[r] : v;
            y[row0 + lane] = (uint16_t)f32_to_bf16_rne(v * scale[row0 + lane]);
        }
        return;
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) part[wv][r] = acc[r];
    }
    __syncthreads();
    if (threadIdx.x < (uint32_t)R && row0 + threadIdx.x < M) {
        float v = 0.f;
        for (uint32_t i = 0; i < W; i++) v += part[i][threadIdx.x];
        y[row0 + threadIdx.x] = (uint16_t)f32_to_bf16_rne(v * scale[row0 + threadIdx.x]);
    }
}

template <int R>
static void launch_fp8_rows(uint32_t jb, dim3 g, dim3 b, hipStream_t st, const uint8_t *w, const float *scale,
                            const float *x, uint16_t *y, uint32_t M, uint32_t K) {
    switch (jb) {
    case 1: hipLaunchKernelGGL((k_fp8_rows<R, 1>), g, b, 0, st, w, scale, x, y, M, K); break;
    case 2: hipLaunchKernelGGL((k_fp8_rows<R, 2>), g, b, 0, st, w, scale, x, y, M, K); break;
    case 3: hipLaunchKernelGGL((k_fp8_rows<R, 3>), g, b, 0, st, w, scale, x, y, M, K); break;
    case 4: hipLaunchKernelGGL((k_fp8_rows<R, 4>), g, b, 0, st, w, scale, x, y, M, K); break;
    case 5: hipLaunchKernelGGL((k_fp8_rows<R, 5>), g, b, 0, st, w, scale, x, y, M, K); break;
    case 6: hipLaunchKernelGGL((k_fp8_rows<R, 6>), g, b, 0, st, w, scale, x, y, M, K); break;
    default: hipLaunchKernelGGL((k_fp8_rows<R, 8>), g, b, 0, st, w, scale, x, y, M, K); break;
    }
}

int launch_ref_fp8(const uint8_t *w, const float *scale, const float *x, uint16_t *y, uint32_t M, uint32_t K, int ncu,
                   hipStream_t st) {
    if ((K & 7u) != 0 || ((uintptr_t)w & 7u) != 0 || ((uintptr_t)x & 15u) != 0) {
        const uint32_t waves = (M + 3) / 4;
        hipLaunchKernelGGL(k_fp8_bytes, dim3((waves + 3) / 4), dim3(256), 0, st, w, scale, x, y, M, K);
        return (int)hipGetLastError();
    }
    // 8 rows per workgroup for tall matrices (at least 4 row groups of 8 per CU), else 4; enough waves per row group
    // that the grid holds about 24 waves per CU, at most one per 512-column chunk and 8 per workgroup.  Sweep on
    // MI355X (R in 2/4/8 x 4-48 waves per CU): gate_up 19456x2560 10.7 us (R 8), lm_head 151936x2560 59.4 us (R 8,
    // 6.6 TB/s), qkv 6144x2560 5.7 us, o 2560x4096 4.9-5.0 us, down 2560x9728 7.9 us (R 4).
    const uint32_t R = M / 8u >= 4u * (uint32_t)ncu ? 8u : 4u, kWavesPerCu = 24u;
    const uint32_t groups = (M + R - 1) / R, J = (K + 511u) / 512u;
    const uint32_t W = std::max(1u, std::min({(kWavesPerCu * (uint32_t)ncu + groups - 1) / groups, J, 8u}));
    const uint32_t jb = std::min(8u, (J + W - 1) / W);
    if (R == 8) launch_fp8_rows<8>(jb, dim3(groups), dim3(64 * W), st, w, scale, x, y, M, K);
    else launch_fp8_rows<4>(jb, dim3(groups), dim3(64 * W), st, w, scale, x, y, M, K);
    return (int)hipGetLastError();
}

// ---- uncompressed BF16 matvec: y = RNE_bf16(W x), W BF16 [M x K] row-major, x BF16 [K] ----
// The k_fp8_rows pattern at two bytes per weight: a workgroup owns R rows, its W waves split each row into chunks of
// 512 columns (chunk j to wave j mod W), lane l owns columns 8l .. 8l + 7 of a chunk: one 16-byte non-temporal load
// per row and one 16-byte load of x (shared by the R rows), JB chunks of every row in flight at once, x first.
// v_dot2_f32_bf16 accumulates pairs in fp32; lane order, then a butterfly over the wave, then the waves in order.
template <int R, int JB>
__global__ void __launch_bounds__(512) k_bf16_rows(const uint16_t *__restrict__ w, const uint16_t *__restrict__ x,
                                                   uint16_t *__restrict__ y, uint32_t M, uint32_t K) {
    __shared__ float part[8][R];
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6, W = blockDim.x >> 6;
    const uint32_t row0 = blockIdx.x * R, J = (K + 511u) >> 9;
    const uint16_t *rp[R];
#pragma unroll
    for (int r = 0; r < R; r++) rp[r] = w + (uint64_t)min(row0 + r, M - 1u) * K;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    for (uint32_t j0 = wv; j0 < J; j0 += W * JB) {
        uint4 q[JB][R], xv[JB];
        bool ok[JB];
        uint32_t cc[JB];
#pragma unroll
        for (int b = 0; b < JB; b++) {
            const uint32_t c = (j0 + b * W) * 512u + 8u * lane;
            ok[b] = j0 + b * W < J && c < K;
            cc[b] = ok[b] ? c : 0u;
            if (JB == 1 || j0 + b * W < J) xv[b] = *(const uint4 *)(x + cc[b]);      // wave-uniform branch
        }
#pragma unroll
        for (int b = 0; b < JB; b++) {
            if (JB == 1 || j0 + b * W < J) {
#pragma unroll
                for (int r = 0; r < R; r++) q[b][r] = ldnt4(rp[r] + cc[b]);
            }
        }
#pragma unroll
        for (int b = 0; b < JB; b++) {
            if (JB > 1 && j0 + b * W >= J) break;
            const uint4 xb = ok[b] ? xv[b] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
            for (int r = 0; r < R; r++) {
                acc[r] = dot2_bf16(q[b][r].x, xb.x, acc[r]);
                acc[r] = dot2_bf16(q[b][r].y, xb.y, acc[r]);
                acc[r] = dot2_bf16(q[b][r].z, xb.z, acc[r]);
                acc[r] = dot2_bf16(q[b][r].w, xb.w, acc[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) part[wv][r] = acc[r];
    }
    __syncthreads();
    if (threadIdx.x < (uint32_t)R && row0 + threadIdx.x < M) {
        float v = 0.f;
        for (uint32_t i = 0; i < W; i++) v += part[i][threadIdx.x];
        y[row0 + threadIdx.x] = (uint16_t)f32_to_bf16_rne(v);
    }
}

// K % 8 != 0 or unaligned pointers: one wave per row, two bytes per lane and step.
__global__ void __launch_bounds__(256) k_bf16_any(const uint16_t *__restrict__ w, const uint16_t *__restrict__ x,
                                                  uint16_t *__restrict__ y, uint32_t M, uint32_t K) {
    const uint32_t lane = threadIdx.x & 63, row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= M) return;
    float acc = 0.f;
    for (uint32_t k = lane; k < K; k += 64) acc = fmaf(bf16_lo(w[(uint64_t)row * K + k]), bf16_lo(x[k]), acc);
    acc = wave_sum(acc);
    if (lane == 0) y[row] = (uint16_t)f32_to_bf16_rne(acc);
}

template <int R>
static void launch_bf16_rows(uint32_t jb, dim3 g, dim3 b, hipStream_t st, const uint16_t *w, const uint16_t *x,
                             uint16_t *y, uint32_t M, uint32_t K) {
    switch (jb) {
    case 1: hipLaunchKernelGGL((k_bf16_rows<R, 1>), g, b, 0, st, w, x, y, M, K); break;
    case 2: hipLaunchKernelGGL((k_bf16_rows<R, 2>), g, b, 0, st, w, x, y, M, K); break;
    case 3: hipLaunchKernelGGL((k_bf16_rows<R, 3>), g, b, 0, st, w, x, y, M, K); break;
    default: hipLaunchKernelGGL((k_bf16_rows<R, 4>), g, b, 0, st, w, x, y, M, K); break;
    }
}

int launch_ref_bf16(const uint16_t *w, const uint16_t *x, uint16_t *y, uint32_t M, uint32_t K, int ncu, hipStream_t st) {
    if ((K & 7u) != 0 || ((uintptr_t)w & 15u) != 0 || ((uintptr_t)x & 15u) != 0) {
        hipLaunchKernelGGL(k_bf16_any, dim3((M + 3) / 4), dim3(256), 0, st, w, x, y, M, K);
        return (int)hipGetLastError();
    }
    // as launch_ref_fp8, with the registers of a chunk in flight doubled (16-byte rows): R = 8 rows per workgroup
    // for tall matrices with at most 2 chunks of each row in flight per wave, otherwise R = 4 with at most 4
    const uint32_t R = M / 8u >= 4u * (uint32_t)ncu ? 8u : 4u, kWavesPerCu = 24u, jb_max = R == 8 ? 2u : 4u;
    const uint32_t groups = (M + R - 1) / R, J = (K + 511u) / 512u;
    const uint32_t W = std::max(1u, std::min({(kWavesPerCu * (uint32_t)ncu + groups - 1) / groups, J, 8u}));
    const uint32_t jb = std::min(jb_max, (J + W - 1) / W);
    if (R == 8) launch_bf16_rows<8>(jb, dim3(groups), dim3(64 * W), st, w, x, y, M, K);
    else launch_bf16_rows<4>(jb, dim3(groups), dim3(64 * W), st, w, x, y, M, K);
    return (int)hipGetLastError();
}

// ---- streaming read: the read bandwidth a launch of a given size reaches ----
// Every workgroup reads a contiguous share of `bytes` (a multiple of 16) with 16-byte non-temporal loads, UNROLL of
// them in flight per thread, folds the words with xor and writes one word: out[blockIdx.x].  The value only keeps
// the loads alive.
template <int UNROLL>
__global__ void __launch_bounds__(256) k_stream_read(const uint4 *__restrict__ p, uint64_t n16, uint32_t *__restrict__ out) {
    const uint64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const uint64_t lo = (uint64_t)blockIdx.x * per, hi = min(lo + per, n16);
    uint32_t v = 0;
    for (uint64_t i = lo + threadIdx.x; i < hi; i += (uint64_t)blockDim.x * UNROLL) {
        uint4 q[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) {
            const uint64_t j = i + (uint64_t)u * blockDim.x;
            q[u] = ldnt4(p + (j < hi ? j : lo));
        }
#pragma unroll
        for (int u = 0; u < UNROLL; u++) v ^= q[u].x ^ q[u].y ^ q[u].z ^ q[u].w;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v ^= (uint32_t)__shfl_xor((int)v, o, 64);
    __shared__ uint32_t red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

int launch_stream_read(const void *p, uint64_t bytes, uint32_t *out, uint32_t grid, hipStream_t st) {
    hipLaunchKernelGGL(k_stream_read<8>, dim3(grid), dim3(256), 0, st, (const uint4 *)p, bytes / 16u, out);
    return (int)hipGetLastError();
}

}  // namespace nwc
