// kern_misc.hip -- the uncompressed fp8 weight-only matvec (the "native fp8" bandwidth baseline the compressed fp8
// path is compared with; counterpart of the reference's kern_ref_fp8, nwc_ops.cu:760-829).
//
// One wave per 4 rows; each lane streams 16 fp8 weights per row per step with a 16-byte non-temporal load,
// converts them with the gfx950 OCP-e4m3 packed conversion (v_cvt_pk_f32_fp8) and accumulates in fp32 against
// fp32 activations.  The wave reduction ends with one BF16 store per row.
#include "nwc_device.h"
#include "nwc_launch.h"

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

__global__ void __launch_bounds__(256) k_ref_fp8(const uint8_t *__restrict__ w, const float *__restrict__ scale,
                                                 const float *__restrict__ x, uint16_t *__restrict__ y, uint32_t M, uint32_t K) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 4;
    if (row0 >= M) return;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    if ((K & 15u) == 0) {
        for (uint32_t k = lane * 16; k < K; k += 64 * 16) {
            float xv[16];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = ((const float4 *)(x + k))[i];
                xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (row0 + r >= M) break;
                const uint4 c = ldnt4((w + (uint64_t)(row0 + r) * K + k));
                const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)cw[j], false);
                    const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)cw[j], true);
                    acc[r] = fmaf(lo.x, xv[4 * j], acc[r]);
                    acc[r] = fmaf(lo.y, xv[4 * j + 1], acc[r]);
                    acc[r] = fmaf(hi.x, xv[4 * j + 2], acc[r]);
                    acc[r] = fmaf(hi.y, xv[4 * j + 3], acc[r]);
                }
            }
        }
    } else {
        for (int r = 0; r < 4; r++) {
            if (row0 + r >= M) break;
            for (uint32_t k = lane; k < K; k += 64) acc[r] = fmaf(fp8_to_f32_exact(w[(uint64_t)(row0 + r) * K + k]), x[k], acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float v = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < M) y[row0 + r] = (uint16_t)f32_to_bf16_rne(v * scale[row0 + r]);
    }
}

int launch_ref_fp8(const uint8_t *w, const float *scale, const float *x, uint16_t *y, uint32_t M, uint32_t K, hipStream_t st) {
    const uint32_t waves = (M + 3) / 4;
    hipLaunchKernelGGL(k_ref_fp8, dim3((waves + 3) / 4), dim3(256), 0, st, w, scale, x, y, M, K);
    return (int)hipGetLastError();
}

}  // namespace nwc
