// nwc_launch.h -- launch plans and the launchers each kernel file exports to the C ABI layer (abi.cpp).
#pragma once
#include "nwc_device.h"

#include <algorithm>

namespace nwc {

struct LaunchPlan {
    int layout;
    bool pipe;              // layout 0: rounds through two region buffers, the next round prefetched
    uint32_t split;         // layout 0: half-waves per block (1, or 2 or 4 with the row index)
    bool seq13;             // layout 0 token path: the 13-bit decode table (a larger static LDS share)
    bool multi;             // layout 1: several items (block, quarter) per half-wave, one 16-row group per workgroup
    uint32_t tail;          // layout 0 token path: k_layout0t, G whole row groups then the rest split tail-ways (2, 4)
    uint32_t grid, threads, lds, G;
    uint32_t slot_words;    // layout 0: region-buffer words per block
};

int launch_prefix(const LaunchPlan &p, int elem_t, int mode, bool xbf16, const BlockArgs &a, hipStream_t st);
int launch_fixed(const LaunchPlan &p, int elem_t, int mode, bool xbf16, const BlockArgs &a, hipStream_t st);
int launch_gather_prefix(int layout, int elem_t, const GatherArgs &a, hipStream_t st);
// layouts 0/1 gather with the row index (k_gather0x / k_gather1x); seq: the 13-bit table or null
int launch_gather0x(int layout, int elem_t, const GatherArgs &a, const uint16_t *aux, const uint32_t *seq, hipStream_t st);
// layout-0 token path for ntok (2..4) activation vectors at once (k_layout0_batch); plan from plan_layout0_batch
int launch_layout0_batch(const LaunchPlan &p, int elem_t, const BlockArgs &a, uint32_t ntok, hipStream_t st);
int launch_gather_fixed(int elem_t, const GatherArgs &a, hipStream_t st);
// layout-0 prefill (k_prefill0): tt tokens per workgroup tile (64, 128, 256 or 512)
int launch_prefill0(int elem_t, uint32_t tt, const PrefillArgs &p, hipStream_t st);
// Y[T x N] = X[T x K] W[N x K]^T (+ bias), BF16 (k_gemm_xwt); the launcher fills nT, S, stages, cnt and part
struct GemmArgs {
    const uint16_t *x, *w, *bias;
    uint16_t *y;
    float *part;            // S partial tiles per output tile (split products)
    uint32_t *cnt;          // per output tile: workgroups of its splits that have finished
    uint32_t ldx, ldw, T, N, K, nT, S, stages;
};
constexpr uint32_t kGemmCounters = 1024;
constexpr uint64_t kGemmScratchBytes = 24ull << 20;     // nwc_gemm_xbf16_noalloc's workspace per GPU
uint32_t gemm_splits(uint32_t T, uint32_t N, uint32_t K, int ncu);
uint64_t gemm_workspace_bytes(uint32_t T, uint32_t N, uint32_t K, int ncu);
int launch_gemm_xwt(GemmArgs g, void *ws, int ncu, hipStream_t st);
// the current device's copy of the library's static workspace (its counters cleared on `st` by the first call on
// the device outside graph capture, and by every captured call before that), or null with *err set
void *gemm_scratch(hipStream_t st, int *err);
int launch_ref_fp8(const uint8_t *w, const float *scale, const float *x, uint16_t *y, uint32_t M, uint32_t K, int ncu,
                   hipStream_t st);
int launch_ref_bf16(const uint16_t *w, const uint16_t *x, uint16_t *y, uint32_t M, uint32_t K, int ncu, hipStream_t st);
int launch_stream_read(const void *p, uint64_t bytes, uint32_t *out, uint32_t grid, hipStream_t st);

}  // namespace nwc
