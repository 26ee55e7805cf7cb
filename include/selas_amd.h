/*
 * selas_amd.h - C ABI of the MI355X (gfx950) NF4 hot path.
 *
 * One shared library, libselas_amd.so, built by hipcc from selas_amd/csrc/.
 * Every entry point:
 *   - takes plain device pointers, element counts and strides (in elements,
 *     not bytes), never a framework type;
 *   - launches asynchronously on the HIP stream passed as `stream` (a
 *     hipStream_t; pass the caller's current stream so that stream-ordered
 *     buffer reuse stays correct) and never synchronises the device;
 *   - allocates nothing and frees nothing: outputs and scratch memory are
 *     caller-owned (a tiled linear whose launch splits its last round of tiles
 *     over K takes a workspace argument, sized by selas_linear_workspace_bytes);
 *   - returns SELAS_OK or an error code and never throws; the message of the
 *     last error on the calling thread is returned by selas_last_error().
 *
 * Data formats follow the reference codec (selas/codecs.py:1-16, 58-63,
 * 86-119): NF4 weights are `packed` uint8 [numel/2] (element 2i in the high
 * nibble of byte i), `absmax` fp32 [numel/blocksize] over the flattened
 * tensor, and a 16-entry fp32 codebook passed by value from host memory
 * (the tensor's meta["code"]); int8_row weights are `q` int8 in the weight's
 * shape and `scale` fp32, one per row.
 *
 * Kernels, tile shapes and K splits are chosen from shapes, dtypes and pointer
 * alignment (and the GPU's CU count) only, never from streams, earlier calls or
 * allocation results, and use no atomics, so equal inputs give equal bits on
 * every call and every stream.
 */
#ifndef SELAS_AMD_H
#define SELAS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes. */
#define SELAS_OK 0
#define SELAS_EINVAL 1       /* invalid argument (sizes, dtypes, nulls): ValueError in the reference */
#define SELAS_EUNSUPPORTED 2 /* valid, but outside what a fused kernel covers: caller falls back */
#define SELAS_EHIP 3         /* HIP runtime or launch error */

/* Element types (the `dtype` arguments). */
#define SELAS_F32 0
#define SELAS_F16 1
#define SELAS_BF16 2

/* Weight codecs (the `codec` argument of selas_linear_workspace_bytes). */
#define SELAS_CODEC_NF4 0
#define SELAS_CODEC_INT8_ROW 1

/* Message of the last failed call on this thread ("" if none). */
const char *selas_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int selas_abi_version(void);

/* ------------------------------------------------------------------ codec */

/*
 * NF4 decode: out[2i]   = dtype(code[packed[i] >> 4] * absmax[i / (blocksize/2)])
 *             out[2i+1] = dtype(code[packed[i] & 15] * absmax[i / (blocksize/2)])
 * The fp32 product is rounded once, to nearest even, to out_dtype; the bits
 * equal the reference decode for every input except NaN payloads.
 * Replaces nf4_dequant / nf4_dequant_torch (selas/codecs.py:178-199, 260-266)
 * and the Triton kernel (codecs.py:207-228).
 */
int selas_nf4_dequant(const uint8_t *packed, const float *absmax, int64_t n_bytes, int64_t blocksize,
                      const float code[16], void *out, int out_dtype, void *stream);

/*
 * NF4 encode of an fp32 tensor of n elements (n % blocksize == 0, blocksize
 * even): absmax[b] = max |w| over block b; each element divided by the block's
 * absmax (1 where absmax is 0) is mapped to the number of codebook midpoints
 * (code[i]+code[i+1])/2 that are not >= it (ties go to the lower code), and
 * two codes are packed per byte, first element high.
 * Replaces encode_nf4 (selas/codecs.py:99-119).
 */
int selas_nf4_encode(const float *w, int64_t n, int64_t blocksize, const float code[16], uint8_t *packed,
                     float *absmax, void *stream);

/*
 * int8_row decode of a weight of `rows` rows of `cols` elements (q int8
 * [rows, cols], scale fp32 [rows]):
 *   out[r, c] = dtype(float(q[r, c]) * float(dtype(scale[r])))
 * i.e. q.to(dtype) * scale.to(dtype) computed in dtype; for bf16 and fp16 the
 * product is exact in fp32 and rounded once. Bit-identical to the reference
 * decode (selas/codecs.py:273-277) except NaN payloads.
 */
int selas_int8_row_dequant(const int8_t *q, const float *scale, int64_t rows, int64_t cols, void *out,
                           int out_dtype, void *stream);

/*
 * int8_row encode of an fp32 weight [rows, cols]: scale[r] = max |w[r, :]| / 127
 * (1 where that max is not positive), q[r, c] = clamp(round_half_even(w[r, c] /
 * scale[r]), -127, 127), with IEEE fp32 division.
 * Replaces encode_int8_row (selas/codecs.py:86-96).
 */
int selas_int8_row_encode(const float *w, int64_t rows, int64_t cols, int8_t *q, float *scale, void *stream);

/* ------------------------------------------------------------ linear */

/*
 * Quantized linear forward y = x W^T + bias with W an NF4 [N, K] weight:
 *   x     [M, K]  dtype, row stride ldx (K contiguous)
 *   bias  [N]     dtype or NULL
 *   y     [M, N]  dtype, row stride ldy
 * dtype is SELAS_BF16 (fp32 accumulation, one rounding of acc + bias).
 * M > 32 runs a tiled MFMA GEMM with the dequantization fused into the operand
 * load; its operand is the reference's decoded weight bf16(code*absmax) bit for
 * bit. M <= 32 runs a skinny dequant-GEMM that multiplies x by the codes and
 * scales the fp32 block sums by absmax (for K = 1024, 2048, 3072 in fp16 after
 * an exact power-of-two rescale of each row of x; otherwise in bf16 with codes
 * split into two bf16 terms); it agrees with the decoded-weight product to the
 * rounding of the decoded weight. Every output of the tiled GEMM sums K in
 * one order, whatever M and the tile height, except where a launch splits its
 * last round of tiles over K (long K and a last round of few tiles, e.g.
 * M 6144, N 3072, K 15360): those tiles' K ranges are summed in fp32 by a
 * second kernel, in a fixed order, from fp32 partial tiles kept in `workspace`
 * (device memory of workspace_bytes >= selas_linear_workspace_bytes for this
 * shape, 16-byte aligned, not read or written by anything else until the
 * launch has run; NULL and 0 where that size is 0, otherwise SELAS_EINVAL).
 * Whether and how a launch splits depends on M, N, K and the CU count only.
 * Returns SELAS_EUNSUPPORTED
 * when the shape or layout is outside the fused kernels (blocksize != 64,
 * K % 64 != 0, misaligned rows, dtype other than bf16); the caller then
 * decodes with selas_nf4_dequant and uses a library GEMM.
 * Replaces UnitView.linear for NF4 weights (selas/store.py:289-293):
 * decode (codecs.py:269-280) followed by F.linear.
 */
int selas_nf4_linear(const void *x, int64_t M, int64_t K, int64_t ldx, const uint8_t *packed,
                     const float *absmax, int64_t blocksize, const float code[16], int64_t N,
                     const void *bias, void *y, int64_t ldy, int dtype, void *workspace, int64_t workspace_bytes,
                     void *stream);

/* At most this many linears per selas_nf4_linear_batched call. */
#define SELAS_MAX_BATCHED_LINEARS 4

/* One quantized linear of a batched launch (host-memory array element); the
 * first fields mean what the arguments of selas_nf4_linear mean.
 * gelu_cols (0 = none) makes the last gelu_cols output columns
 * y2[m, j] = bf16(gelu_tanh(bf16(x W^T + b)[m, N - gelu_cols + j])) instead, with
 * row stride ldy2: the GELU that follows the block's MLP input linears
 * (flux.py:194-200), applied to the rounded output exactly as a separate GELU
 * kernel would. N - gelu_cols must be a multiple of 256; with gelu_cols = N, y
 * is not written and may be NULL. */
typedef struct selas_nf4_gemm_problem {
  const void *x;
  int64_t M, K, ldx;
  const uint8_t *packed;
  const float *absmax;
  int64_t N;
  const void *bias;
  void *y;
  int64_t ldy;
  void *y2;
  int64_t ldy2, gelu_cols;
} selas_nf4_gemm_problem;

/*
 * Up to SELAS_MAX_BATCHED_LINEARS independent quantized linears (each its own
 * x, weight, bias and y; all M > 32) in one launch of the tiled GEMM: the
 * tiles of all problems share the GPU, so a small problem fills the CUs a
 * large one leaves idle in its last round. Each y has the bits
 * selas_nf4_linear gives for that problem alone, except in tiles that the
 * batch's launch splits over K (the plan, like the workspace it needs, depends
 * on all the problems' shapes: e.g. 4096- and 2048-token problems of
 * K 12288 together leave a last round of few tiles that neither leaves alone).
 * workspace / workspace_bytes as for selas_nf4_linear, sized by
 * selas_linear_workspace_bytes over the same problems. Returns SELAS_EUNSUPPORTED,
 * launching nothing, when any problem is outside the tiled GEMM (M <= 32 or
 * any reason selas_nf4_linear would give); the caller then runs them one by one.
 * No counterpart in the reference: it replaces consecutive UnitView.linear
 * calls on independent inputs, e.g. the image and text streams of FLUX's
 * double block (selas/models/flux.py:300-324).
 */
int selas_nf4_linear_batched(const selas_nf4_gemm_problem *problems, int64_t count, int64_t blocksize,
                             const float code[16], int dtype, void *workspace, int64_t workspace_bytes,
                             void *stream);

/*
 * Bytes of device workspace that selas_nf4_linear (count 1) or
 * selas_nf4_linear_batched (codec SELAS_CODEC_NF4), or their int8_row twins
 * (SELAS_CODEC_INT8_ROW), need for these problems on the current device:
 * 0 unless the launch splits its last round of tiles over K, then
 * split tiles x K ranges x 256 KiB (at most the CU count x 256 KiB, 64 MiB on
 * MI355X). Reads only M, K and N of each problem (the other fields may be
 * NULL); problems with M = 0 are skipped, and M <= 32 gives 0 (skinny kernels).
 * No counterpart in the reference: selas's decode-then-F.linear needs no
 * scratch beyond the decoded weight (selas/store.py:289-293).
 */
int selas_linear_workspace_bytes(const selas_nf4_gemm_problem *problems, int64_t count, int codec,
                                 int64_t *bytes);

/*
 * Quantized linear forward y = x W^T + bias with W an int8_row [N, K] weight
 * (q int8 [N, K] row-major, 16-byte aligned; scale fp32 [N]); x, bias, y and
 * dtype as for selas_nf4_linear.
 * M > 32 runs the tiled MFMA GEMM of selas_nf4_linear with the int8 operand
 * bf16(q * bf16(scale)), the reference's decoded weight bit for bit. M <= 32
 * runs a skinny kernel (for K = 1024, 2048, 3072 the streaming kernel of
 * selas_int8_row_linear_grouped) that multiplies x by q exactly and scales the fp32 row
 * sums by bf16(scale): it agrees with the decoded-weight product to the bf16
 * rounding of the decoded weight. workspace / workspace_bytes as for
 * selas_nf4_linear (selas_linear_workspace_bytes with SELAS_CODEC_INT8_ROW).
 * Returns SELAS_EUNSUPPORTED for K % 64 != 0,
 * misaligned rows or a dtype other than bf16 (the caller then decodes with
 * selas_int8_row_dequant and uses a library GEMM).
 * Replaces UnitView.linear for int8_row weights (selas/store.py:289-293):
 * decode (codecs.py:273-277) followed by F.linear.
 */
int selas_int8_row_linear(const void *x, int64_t M, int64_t K, int64_t ldx, const int8_t *q, const float *scale,
                          int64_t N, const void *bias, void *y, int64_t ldy, int dtype, void *workspace,
                          int64_t workspace_bytes, void *stream);

/*
 * selas_nf4_linear_batched for int8_row weights: in each problem `packed`
 * holds q and `absmax` the row scales; gelu_cols, y2 and the workspace as
 * there (selas_linear_workspace_bytes with SELAS_CODEC_INT8_ROW).
 * No counterpart in the reference (see selas_nf4_linear_batched).
 */
int selas_int8_row_linear_batched(const selas_nf4_gemm_problem *problems, int64_t count, int dtype, void *workspace,
                                  int64_t workspace_bytes, void *stream);


/*
 * One NF4 weight of a grouped skinny linear (device-memory array element).
 * packed/absmax as for selas_nf4_linear, bias [n] bf16 or NULL, y [M, n] bf16
 * with row stride ldy. The layout is fixed: 4 pointers then 2 int64.
 */
typedef struct selas_nf4_gemv_desc {
  const uint8_t *packed;
  const float *absmax;
  const void *bias;
  void *y;
  int64_t n;
  int64_t ldy;
} selas_nf4_gemv_desc;

/*
 * `count` quantized linears that share one input x [M, K] (M <= 32, K = 1024,
 * 2048 or 3072, blocksize 64, bf16, at most 1023 weights, 16-byte aligned codes
 * and x rows, x spanning under 4 GiB), computed by one launch: y_i = x W_i^T + b_i.
 * `descs` is a device array of `count` descriptors and total_n the sum of
 * their n (it sizes the launch). Each output has the bits selas_nf4_linear
 * gives for that weight alone.
 * Replaces the per-unit loop of FluxRunner.modulations (selas/models/flux.py:
 * 428-445), which calls UnitView.linear once per modulation weight with the
 * same silu(vec) input.
 */
int selas_nf4_linear_grouped(const void *x, int64_t M, int64_t K, int64_t ldx, const selas_nf4_gemv_desc *descs,
                             int64_t count, int64_t total_n, int64_t blocksize, const float code[16], int dtype,
                             void *stream);

/* At most this many weights per selas_nf4_linear_grouped_static call. */
#define SELAS_STATIC_MAX_WEIGHTS 1023
/* At most this many streams per GPU call selas_nf4_linear_grouped_static. */
#define SELAS_STATIC_MAX_STREAMS 8

/*
 * selas_nf4_linear_grouped that allocates nothing and needs no device memory of
 * the caller's beyond x, the weights, biases and outputs: `descs` is an array
 * of `count` descriptors in HOST memory (read during the call only), and the
 * sum of their n is computed here. The library stages the descriptors in
 * device tables of its own: SELAS_STATIC_MAX_STREAMS tables of
 * SELAS_STATIC_MAX_WEIGHTS * 48 bytes (392,832 bytes in all) per GPU, held until
 * the process ends. Each stream that calls on a GPU gets its own table, at its
 * first call; a call from a further stream returns SELAS_EUNSUPPORTED, and
 * count above SELAS_STATIC_MAX_WEIGHTS is rejected with SELAS_EINVAL. A call
 * rewrites its stream's table before its kernels read it, and enqueues both
 * under that table's lock: calls on one stream are ordered (also from several
 * host threads), and calls on different streams use different tables. A
 * stream handle that is destroyed and handed out again keeps the old table, so
 * the destroyed stream's calls must have finished. Each output has the bits
 * selas_nf4_linear_grouped (and selas_nf4_linear) gives for that weight.
 * No counterpart in the reference. It is for callers that cannot allocate
 * device memory: code under HIP graph capture, serving loops with a fixed
 * memory budget, harnesses that forbid hipMalloc.
 */
int selas_nf4_linear_grouped_static(const void *x, int64_t M, int64_t K, int64_t ldx, const selas_nf4_gemv_desc *descs,
                                    int64_t count, int64_t blocksize, const float code[16], int dtype, void *stream);

/*
 * selas_nf4_linear_grouped for int8_row weights (M <= 32, K = 1024, 2048 or
 * 3072, bf16, 16-byte aligned x rows, x spanning under 4 GiB): in each
 * descriptor `packed` holds q [n, K] (16-byte aligned) and
 * `absmax` the n row scales. Each output has the bits selas_int8_row_linear
 * gives for that weight alone (the same kernel serves M <= 32 there).
 * Replaces the per-weight UnitView.linear calls of FluxRunner.modulations
 * (selas/models/flux.py:428-445) for int8_row weights.
 */
int selas_int8_row_linear_grouped(const void *x, int64_t M, int64_t K, int64_t ldx, const selas_nf4_gemv_desc *descs,
                                  int64_t count, int64_t total_n, int dtype, void *stream);

/* ------------------------------------------------------------ segments
 *
 * The memory-bound code between the block linears (selas/models/flux.py:
 * 164-200). Tensors are [B, L, D] with D contiguous; `sb`/`sl` are the batch
 * and row strides in elements. Per-batch vectors (shift, scale, gate) are
 * [B, D] with batch stride `mod_sb`. Outputs are contiguous. All math is fp32.
 */

/* out = dtype(LayerNorm(x; no affine, eps 1e-6) * (1 + scale) + shift).
 * Replaces _mod_in (flux.py:164-166) with _ln (flux.py:146-147). */
int selas_mod_in(const float *x, int64_t B, int64_t L, int64_t D, int64_t x_sb, int64_t x_sl,
                 const float *shift, const float *scale, int64_t mod_sb, void *out, int out_dtype,
                 void *stream);

/* out = x + g * float(y), y clamped to +-65504 first when guard != 0.
 * Replaces _gated_add (flux.py:169-171) with _res (flux.py:141-143). */
int selas_gated_add(const float *x, int64_t B, int64_t L, int64_t D, int64_t x_sb, int64_t x_sl,
                    const float *g, int64_t g_sb, const void *y, int y_dtype, int64_t y_sb, int64_t y_sl,
                    int guard, float *out, void *stream);

/* x_out = x + g * float(y) as above, and h = mod_in(x_out, shift, scale) in one pass.
 * Replaces _gated_add_mod (flux.py:174-176). */
int selas_gated_add_mod(const float *x, int64_t B, int64_t L, int64_t D, int64_t x_sb, int64_t x_sl,
                        const float *g, int64_t g_sb, const void *y, int y_dtype, int64_t y_sb, int64_t y_sl,
                        int guard, const float *shift, const float *scale, int64_t mod_sb, float *x_out,
                        void *h, int h_dtype, void *stream);

/* Single-stream attention prep: qkv [B, L, 3*H*Dh] (channel = which*H*Dh + h*Dh + d,
 * strides qkv_sb, qkv_sl) -> q, k = dtype(RoPE(RMSNorm(.) * scale)), v = copy,
 * each [B, H, L, Dh] contiguous. RMSNorm eps 1e-6 over Dh in fp32; RoPE rotates
 * interleaved pairs with cos/sin [L, Dh/2] fp32. Dh must be even and at most 128.
 * Replaces _qkv_single (flux.py:188-191) with _heads, qk_rms, apply_rope (117-132). */
int selas_qkv_single(const void *qkv, int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t qkv_sb,
                     int64_t qkv_sl, const float *q_scale, const float *k_scale, const float *cos,
                     const float *sin, void *q, void *k, void *v, int dtype, void *stream);

/* Double-stream attention prep: text qkv [B, Lt, 3HDh] and image qkv [B, Li, 3HDh],
 * each normalised with its own q/k scales, joined text-first along L, RoPE with
 * cos/sin [Lt+Li, Dh/2]; q, k, v [B, H, Lt+Li, Dh] contiguous.
 * Replaces _qkv_double (flux.py:179-185). */
int selas_qkv_double(const void *tqkv, int64_t t_sb, int64_t t_sl, int64_t Lt, const void *iqkv, int64_t i_sb,
                     int64_t i_sl, int64_t Li, int64_t B, int64_t H, int64_t Dh, const float *tq_scale,
                     const float *tk_scale, const float *iq_scale, const float *ik_scale, const float *cos,
                     const float *sin, void *q, void *k, void *v, int dtype, void *stream);

/* out = gelu_tanh(h) for rows x cols (row stride ld), out contiguous.
 * Replaces _gelu (flux.py:194-195). */
int selas_gelu(const void *h, int64_t rows, int64_t cols, int64_t ld, void *out, int dtype, void *stream);

/* out[r] = concat(attn[r] (Da), gelu_tanh(mlp[r]) (Dm)), out [rows, Da+Dm] contiguous.
 * Replaces _attn_mlp (flux.py:198-200). */
int selas_attn_mlp(const void *attn, int64_t rows, int64_t Da, int64_t lda, const void *mlp, int64_t Dm,
                   int64_t ldm, void *out, int dtype, void *stream);

/* ------------------------------------------------------------ attention
 *
 * The block attention (selas/models/flux.py:135-138): SDPA over q, k, v
 * [B, H, L, Dh] followed by transpose(1, 2).reshape(B, L, H*Dh).
 */

/*
 * out[b, l, h*Dh + d] = sum_j softmax_j(q[b,h,l,:] . k[b,h,j,:] / sqrt(Dh)) v[b,h,j,d]
 * with q, k [B, H, L, Dh] contiguous, the values given transposed as vt
 * [B, H, Dh, Lp] (selas_transpose_heads; Lp = L rounded up to a multiple of 64,
 * the columns past L zero), out [B, L, H*Dh] with row stride ldo
 * (>= H*Dh; e.g. the first columns of the [attention | GELU(mlp)] input of the
 * single block's second linear, flux.py:198-200). bf16 in
 * and out; scores, softmax and sums in fp32, the probabilities rounded to bf16
 * for the second product (as the flash backends of torch's SDPA do). Takes
 * Dh = 128 and any L; otherwise SELAS_EUNSUPPORTED (the caller runs SDPA).
 * Replaces _attention (flux.py:135-138).
 */
int selas_attention(const void *q, const void *k, const void *vt, int64_t B, int64_t H, int64_t L, int64_t Dh,
                    void *out, int64_t ldo, int dtype, void *stream);

/*
 * vt[i, d, l] = v[i, l, d] for BH heads of [L, Dh] (bf16, Dh = 128), with vt rows
 * of Lp = L rounded up to a multiple of 64 tokens and vt[i, d, l] = 0 for l >= L:
 * the value layout selas_attention reads. No counterpart in the reference.
 */
int selas_transpose_heads(const void *v, int64_t BH, int64_t L, int64_t Dh, void *vt, int dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SELAS_AMD_H */
