/* nwc_oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C, serial restatement of the NWC v9/v10/v11 format (the encoder, the lookup-table builder and a
 * bit-serial decoder for all three layouts and both element types) plus an fp32 CPU matvec.  It is the
 * checker the tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP library with.
 * Nothing in the product (nwc_amd/) links, imports or calls it.
 *
 * Reference followed (parda21/NWC): csrc/nwc_ops.cu:48-348 (constants, Shape, planes, encoders, LUT),
 * :407-442 / :552-565 / :832-879 (what the kernels decode), tests/test_format_cpu.py:14-111 (the reference's
 * own CPU decoder), docs/format.md sections 2-4d.  Each function below cites the lines it restates.
 */
#ifndef NWC_ORACLE_H
#define NWC_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* nwc_ops.cu:121-126: [blocks, raw-plane bytes, scratch floats, K16]; -1 on M == 0, K == 0, M > 2^32-1 */
int or_layout(uint64_t M, uint32_t K, int elem, uint64_t *out);

/* nwc_ops.cu:245-320 (layouts 0/1) and :175-243 (layout 2).  Same buffers and return codes as nwc_encode:
 * data length incl. 64 B slack, -1 shape/capacity, -2 NaN in fp8, -3 layout-2 lane with > 255 exceptions.
 * Unlike the reference, every byte of data[0 .. return) that is not a stream word is written as zero. */
int64_t or_encode(const void *w, uint64_t n, uint32_t K, int elem, uint16_t *freq, uint16_t *psym,
                  uint32_t *bases, uint8_t *hdr, uint8_t *data, uint64_t data_cap, uint8_t *low);

/* nwc_ops.cu:324-348 */
void or_build_tab(const uint16_t *psym, int elem, uint32_t *lut);

/* Bit-serial decoder (test_format_cpu.py:36-111 for BF16; the fp8 assembly of nwc_ops.cu:418-442 / :836-879).
 * out = BF16 bits [M x K] (fp8: the unscaled fp8 value as BF16, exact).  Returns 0, or a negative code when the
 * stream is malformed (OpenMP over row groups, `threads` of them when > 0): -1 read past data_len, -2 filler weight not coded as rank 0 / sign 0, -3 planes of a
 * filler or an exception not zero, -4 duplicate or unused exception entry, -5 bad shape. */
int or_decode(const uint8_t *data, uint64_t data_len, const uint32_t *bases, const uint8_t *hdr, const uint32_t *lut,
              const uint8_t *low, uint64_t M, uint32_t K, int elem, uint16_t *out, int threads);

/* y[m] = sum_k bf16(w[m,k]) * x[k], fp32 accumulation in ascending k, OpenMP over rows (threads <= 0: all). */
void or_matvec_f32(const uint16_t *w, uint64_t M, uint32_t K, const float *x, float *y, int threads);

/* End to end on the compressed tensors (the CPU baseline): decode one row group at a time (all its column
 * blocks) into a private tile, then the fp32 matvec of or_matvec_f32, times scale[m] if scale != NULL.
 * OpenMP over row groups.  Returns 0 or the or_decode error code. */
int or_linear(const uint8_t *data, uint64_t data_len, const uint32_t *bases, const uint8_t *hdr, const uint32_t *lut,
              const uint8_t *low, uint64_t M, uint32_t K, int elem, const float *x, const float *scale, float *y,
              int threads);

/* Closed-form fp8 e4m3fn (OCP, bias 7, no infinities, 0x7F/0xFF = NaN) round-to-nearest-even of an fp32 that is
 * already clamped to +-448 (nwc_torch.py:88-94 clamps before .to(float8_e4m3fn)). */
uint8_t or_f32_to_e4m3(float v);
/* fp8 e4m3fn byte -> fp32, from the definition (e >= 1: 2^(e-7) (1 + m/8); e = 0: m 2^-9). */
float or_e4m3_to_f32(uint8_t b);
/* or_f32_to_e4m3 over an array (OpenMP; threads <= 0: all). */
void or_quantize_e4m3(const float *v, uint64_t n, uint8_t *out, int threads);

/* The fp8 split tables (nwc_ops.cu:140-148, :165-173) exposed for the exhaustive known-answer tests. */
int or_fp8_split(uint8_t b, uint8_t *sym, uint8_t *nib);
int or_fp8_split2(uint8_t b, uint8_t *sym, uint8_t *m3);
uint8_t or_fp8_hb2(int sym);
uint8_t or_fp8_lb2(int sym);
/* nwc_ops.cu:159-160: layout 1/2 lane/stream position -> row offset (0..15) and column offset (0..31) */
uint32_t or_frag_row(uint32_t lane, uint32_t i);
uint32_t or_frag_col(uint32_t lane, uint32_t i);

#ifdef __cplusplus
}
#endif
#endif
