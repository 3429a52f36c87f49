/* nwc_ops.h -- the C ABI of libnwc_ops.so for AMD Instinct MI355X (gfx950).
 *
 * A drop-in for the reference library parda21/NWC csrc/nwc_ops.cu (exports listed at nwc_ops.cu:27-39 and
 * docs/format.md:176-188): the same symbol names, argument order, argument meaning and return codes, so the
 * reference's ctypes bindings (nwc/nwc_torch.py:58-77) load this library unchanged.  Every pointer is a plain
 * address; `stream` is a hipStream_t passed as void* (torch.cuda.current_stream().cuda_stream), work is ordered on
 * it and no entry point synchronises the host.  The library allocates no device memory: outputs, the scratch
 * buffer and workspaces belong to the caller (nwc_gemm_xbf16_noalloc uses a static array of the library instead).
 * `elem` = element type (0 BF16, 1 fp8 e4m3fn) | layout << 4 (layouts 0, 1, 2).
 * `block` must be 4096 (nwc_info(4)); K is the number of columns, n = M * K.
 *
 * This build's extension of `elem` (no counterpart in the reference, whose callers leave these bits zero): bits
 * 8-15 = S / 16 for a layout-0 or layout-1 matrix whose block streams sit in fixed slots of S bytes (a multiple of
 * 16, 16 <= S <= 1728 for layout 0 and <= 3040 for layout 1): block b's lane streams start at byte b * S of `data`,
 * bases[b] == b * S, and `data` holds nb * S + 128 bytes (the slots' padding and the tail zero).  Such tensors are
 * still a valid tensor set of the format; the bits only let the token kernels compute a block's offset instead of
 * reading bases[b] before they can request its streams.  A caller that sets them for tensors that do not meet this
 * contract makes the kernels read the wrong bytes.  The bits are refused (-1) for layout 2, for S above the layout's
 * limit, or when nb * S + 128 >= 2^32.
 *
 * Device entry points return 0, -1 for a shape the format cannot describe (or, in this build, a raw plane the
 * kernels cannot address with 32-bit offsets: layout 0 with Mp * K16 >= 2^32 for Mp = M rounded up to 8 rows,
 * layouts 1/2 with a plane of 2^32 - 512 bytes or more), or a hipError_t code of the launch.  `low` must be followed by the format's 512
 * slack bytes (nwc_torch.py:43); the kernels read into them.  Activations (x, and the batched and prefill x
 * matrices) must be 16-byte aligned: the kernels read them in 16-byte pieces (nwc_ref_fp8 and nwc_ref_bf16 accept
 * any alignment).
 */
#ifndef NWC_OPS_H
#define NWC_OPS_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Capability query.  0: format version (11), 1: states per lane (1), 2: table words (4096), 3: header bytes per
 * block (32), 4: block size (4096), 5: elem parameter present (1), 6: layout 1 supported (1), 7: layout 2
 * supported (1), other: -1.  Replaces nwc_ops.cu:100-106. */
int nwc_info(int what);

/* out[0..3] = [blocks, bytes of the raw plane `low` (without slack), scratch floats (Mp * CB), K16];
 * -1 if M == 0, K == 0 or M > 2^32 - 1.  Replaces nwc_ops.cu:121-126. */
int nwc_layout(uint64_t M, uint32_t K, int elem, uint64_t *out);

/* Host encoder.  w: BF16 bits (uint16 [n]) or fp8 e4m3fn bytes (uint8 [n]), row-major M x K.  Writes
 * psym[0..1023] (exp_of_rank / layout-2 rank tables), bases[nb], hdr[32 nb], data[.. return value), low[raw bytes];
 * freq[0..1023] is cleared.  Returns the data length including 64 bytes of read-ahead slack, -1 for a bad shape,
 * insufficient capacity or a lane stream longer than 255 words, -2 for NaN in fp8 input, -3 for a layout-2 lane with
 * more than 255 exceptions.  Output bytes equal the reference encoder's.  Replaces nwc_ops.cu:245-320 (and
 * encode2, :175-243). */
int64_t nwc_encode(const void *w, uint64_t n, uint32_t K, int elem, uint16_t *freq, uint16_t *psym, uint32_t *bases,
                   uint8_t *hdr, uint8_t *data, uint64_t data_cap, uint8_t *low);

/* Host: the 4096-word decode table from psym (layout 2: the 4-word rank tables).  Replaces nwc_ops.cu:324-348. */
void nwc_build_tab(const uint16_t *freq, const uint16_t *psym, int elem, uint32_t *lut);

/* fp32 test path y[M] = W x; x fp32 [K16] (zero beyond K; layouts 1/2: [K32]).  Unlike the reference (memset +
 * atomics, nwc_ops.cu:1110-1118) every y[m] is written exactly once, so no clearing is needed and the result is
 * deterministic.  Replaces nwc_ops.cu:1110. */
int nwc_matvec(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
               const uint8_t *low, const float *x, float *y, uint64_t n, uint32_t block, uint32_t K, int elem);

/* Decompression to BF16 [M x K16], row stride K16 (fp8: the unscaled fp8 values, exact in BF16).
 * Replaces nwc_ops.cu:1121. */
int nwc_dequant(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                const uint8_t *low, uint16_t *out, uint64_t n, uint32_t block, uint32_t K, int elem);

/* nwc_dequant with the row index from nwc_row_index (layouts 0/1, device; NULL: none) and the 13-bit decode table from
 * nwc_seq_table (device; layouts 0/1; NULL: none), block fixed at 4096.  With the index, small matrices split each
 * block over two or four half-waves; with the table, fewer decode steps take the slow path.  Same output.
 * No counterpart in the reference. */
int nwc_dequant_seq(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                    const uint8_t *low, const uint16_t *row_index, const uint32_t *seq_table, uint16_t *out, uint64_t n,
                    uint32_t K, int elem);

/* Token path y = RNE_bf16(scale * (W x) + bias).  x: layout 0 fp32 [K16], layouts 1/2 BF16 [K32] (zero beyond K),
 * passed through a float pointer as in the reference; bias BF16 [M] or NULL; scale fp32 [M] or NULL (fp8);
 * scratch fp32 [Mp * CB] is accepted for ABI compatibility and not touched (the column-block partial sums are
 * reduced inside the kernel); y BF16 [M].  Replaces nwc_ops.cu:1130. */
int nwc_linear_bf16(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                    const uint8_t *low, const float *x, const uint16_t *bias, const float *scale, float *scratch,
                    uint16_t *y, uint64_t n, uint32_t block, uint32_t K, int elem);

/* Token path with x as BF16 for every layout (layout 0: BF16 [K16]; layouts 1/2: BF16 [K32]), otherwise as
 * nwc_linear_bf16.  row_index: the row index from nwc_row_index, or NULL; with it, small matrices decode each block
 * on two or four half-waves at once (same results).  seq_table: the 13-bit decode table of layouts 0/1 from
 * nwc_seq_table (device, 8196 words), or NULL; with it fewer decode steps take the slow path (same results).  No counterpart in
 * the reference, whose Python side converts x to fp32 for layout 0 with an extra kernel (nwc_torch.py:238-239);
 * callers that hold BF16 activations use this one. */
int nwc_linear_xbf16(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                     const uint8_t *low, const uint16_t *row_index, const uint32_t *seq_table, const uint16_t *x,
                     const uint16_t *bias, const float *scale, uint16_t *y, uint64_t n, uint32_t K, int elem);

/* Token path for ntok = 1..4 activation vectors at once, layout 0 (small batches): x BF16 [ntok][K16], y BF16
 * [ntok][M], bias/scale as nwc_linear_bf16; seq_table as in nwc_linear_xbf16 (NULL: the stored 12-bit LUT).  Every
 * decoded weight is multiplied into the ntok sums, so the matrix is decoded and read once for all of them; y[t] is
 * bit-identical to nwc_linear_xbf16 on x[t].  -1 for layouts 1/2, ntok outside 1..4, or a matrix wider than
 * 16384 columns.  No counterpart in the reference, whose Python side decompresses the whole matrix to a temporary
 * BF16 buffer for any input of more than one token (nwc_torch.py:320-323). */
int nwc_linear_xbf16_batch(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr,
                           const uint32_t *tab, const uint8_t *low, const uint32_t *seq_table, const uint16_t *x,
                           const uint16_t *bias, const float *scale, uint16_t *y, uint64_t n, uint32_t K, int elem,
                           uint32_t ntok);

/* Prefill of a layout-0 matrix for ntok >= 1 tokens without a temporary BF16 matrix: x BF16 [ntok][K16] (columns past
 * K zero), y BF16 [ntok][M] = W x[t] (fp8: times scale) + bias, accumulated in fp32 on the matrix cores (summation order
 * differs from a GEMM library's: results agree with F.linear on the decompressed weights to fp32 rounding, not bit for
 * bit).  Each workgroup decodes 64 rows x 512 columns into LDS once per tile of up to 256 tokens.  row_index (from
 * nwc_row_index) and seq_table (from nwc_seq_table) are required.  0 for ntok = 0; -1 for layouts 1/2, a missing
 * row_index or seq_table, or ntok above 4194240.  Replaces the reference's prefill path, nwc_dequant into a temporary
 * BF16 buffer + F.linear (nwc_torch.py:320-323, nwc_ops.cu:1121-1126); no counterpart export. */
int nwc_prefill_xbf16(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                      const uint8_t *low, const uint16_t *row_index, const uint32_t *seq_table, const uint16_t *x,
                      const uint16_t *bias, const float *scale, uint16_t *y, uint64_t n, uint32_t K, int elem,
                      uint32_t ntok);

/* Host: the 13-bit token-path decode table of layouts 0/1 from a stored LUT (host copy of `tab`): out[0..8191] one entry
 * per 13-bit window that starts with two complete codes ((16 - bits) | byte0 << 8 | byte1 << 16) or 0x40000000,
 * out[8192..8195] exp_of_rank[0..15].  Derived from the stored tensors once per matrix, not part of the format; 0,
 * or -1 for layout 2.  No counterpart in the reference. */
int nwc_seq_table(const uint32_t *lut, int elem, uint32_t *out);

/* Layout-0 row index of a matrix: row_index[(b * 3 + j) * 32 + L] = the bit position, from lane L's first stream word
 * of block b, where row 2 (j + 1) begins (uint16 [blocks x 3 x 32], 192 bytes per block).  Derived from the stored
 * tensors (it is not part of the format), once per matrix; -1 for layouts 1/2 or a bad shape.  No counterpart in
 * the reference. */
int nwc_row_index(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                  const uint8_t *low, uint16_t *row_index, uint64_t n, uint32_t K, int elem);

/* Half-waves per block that nwc_linear_xbf16 would use on the current device (1, or 2 or 4 with a row index), for byte
 * accounting; with_row_index: bit 0 = a row index is passed, bit 1 = the 13-bit table is passed (plans differ with
 * it); -1 for a bad shape.  No counterpart in the reference. */
int nwc_token_split(uint64_t n, uint32_t K, int elem, int with_row_index);

/* Rows ids[0..n_ids) -> BF16 [n_ids x K16] (embedding lookup from the compressed matrix); ids outside [0, M) leave
 * their output row untouched, as in the reference.  0 for n_ids == 0.  Replaces nwc_ops.cu:1143. */
int nwc_gather(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
               const uint8_t *low, const int64_t *ids, uint32_t n_ids, uint16_t *out, uint64_t n, uint32_t block,
               uint32_t K, int elem);

/* nwc_gather for layouts 0/1 with the row index (from nwc_row_index) and, optionally, the 13-bit table (nwc_seq_table;
 * NULL: the stored LUT).  Layout 0: decoding starts at the row pair that holds each row, so a lookup decodes at most
 * two rows of each block instead of up to eight.  Layout 1: four half-waves per block, each from the index's start of
 * its quarter of the super-chunks.  Same output, bit for bit; ids outside [0, M) leave their row untouched.  -1 for
 * layout 2, a missing row_index or a bad shape; 0 for n_ids == 0.  No counterpart in the reference (its lookup is
 * nwc_gather, nwc_ops.cu:1143). */
int nwc_gather_xindex(void *stream, const uint8_t *data, const uint32_t *bases, const uint8_t *hdr, const uint32_t *tab,
                      const uint8_t *low, const uint16_t *row_index, const uint32_t *seq_table, const int64_t *ids,
                      uint32_t n_ids, uint16_t *out, uint64_t n, uint32_t K, int elem);

/* Uncompressed fp8 weight-only matvec (the bandwidth baseline): y = RNE_bf16(scale * (W8 x)), w fp8 e4m3fn [M x K]
 * row-major, scale fp32 [M], x fp32 [K16], y BF16 [M].  Replaces nwc_ops.cu:1163. */
int nwc_ref_fp8(void *stream, const uint8_t *w, const float *scale, const float *x, uint16_t *y, uint64_t M, uint32_t K);

/* Uncompressed BF16 matvec (a bandwidth baseline next to hipBLASLt): y = RNE_bf16(W x), w BF16 [M x K] row-major, x
 * BF16 [K], y BF16 [M], fp32 accumulation.  No counterpart in the reference (its BF16 bar is cuBLAS through F.linear). */
int nwc_ref_bf16(void *stream, const uint16_t *w, const uint16_t *x, uint16_t *y, uint64_t M, uint32_t K);

/* Bytes of workspace nwc_gemm_xbf16 needs for this product on the current device (0: none). */
uint64_t nwc_gemm_workspace(uint32_t T, uint32_t N, uint32_t K);

/* Prefill product of a dequantized matrix: y[t][n] = RNE_bf16(sum_k x[t][k] w[n][k] + bias[n]) for t < T, n < N;
 * x BF16 [T x K] with row stride ldx, w BF16 [N x K] with row stride ldw (nwc_dequant_seq's output, ldw = K16), bias
 * BF16 [N] or null, y BF16 [T x N] row-major; fp32 accumulation on the matrix cores.  K a multiple of 64, ldx and
 * ldw multiples of 8, x and w 16-byte aligned, y 8-byte aligned.  When nwc_gemm_workspace(T, N, K) > 0 the columns
 * are split over several workgroups per output tile: `ws` (256-byte aligned, ws_bytes at least that) holds their
 * partial sums, and its first 4096 bytes are counters that must be zero before the first call on a buffer (every
 * call leaves them zero).  Calls that share a workspace must not overlap (order them on one stream).  The partial
 * sums are added in a fixed order, so a call's result does not depend on the timing.  Replaces the cuBLAS GEMM of
 * the reference's prefill (nwc/nwc_torch.py:320-323: F.linear on the dequantized matrix); no ABI counterpart. */
int nwc_gemm_xbf16(void *stream, const uint16_t *x, uint32_t ldx, const uint16_t *w, uint32_t ldw,
                   const uint16_t *bias, uint16_t *y, uint32_t T, uint32_t N, uint32_t K, void *ws, uint64_t ws_bytes);

/* nwc_gemm_xbf16 without the workspace arguments, for callers that cannot allocate device memory (code under graph
 * capture, tight serving loops, harnesses that forbid hipMalloc); no counterpart in the reference.  The partial sums
 * live in a static array of the library, 24 MiB on each GPU it runs on, held until the process ends (its counters
 * are cleared by a small kernel on `stream` at the first call on a device outside graph capture, and by every
 * captured call before that one).  A product whose workspace would exceed 24 MiB returns -1.  Every call on one GPU
 * shares that array, so calls that overlap on one GPU (two streams) race.  Allocates nothing; same results as
 * nwc_gemm_xbf16. */
int nwc_gemm_xbf16_noalloc(void *stream, const uint16_t *x, uint32_t ldx, const uint16_t *w, uint32_t ldw,
                           const uint16_t *bias, uint16_t *y, uint32_t T, uint32_t N, uint32_t K);

/* Measurement kernel: `grid` workgroups read p[0 .. bytes) once (16-byte non-temporal loads, bytes a multiple of 16,
 * p 16-byte aligned) and write one folded word each to out[0 .. grid).  The read bandwidth a launch of that size
 * reaches.  No counterpart in the reference. */
int nwc_stream_read(void *stream, const void *p, uint64_t bytes, uint32_t *out, uint32_t grid);

/* Device set-up; returns the compute-unit count of the current device (0 without a usable GPU).  Called lazily by
 * the launchers.  Replaces nwc_ops.cu:1170. */
int nwc_setup(void);

#ifdef __cplusplus
}
#endif
#endif
