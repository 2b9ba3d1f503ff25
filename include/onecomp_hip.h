/*
 * onecomp_hip.h - C ABI of the MI355X (gfx950) int4 dequant + GEMM library
 * (libonecomp_hip.so).
 *
 * Every entry point is `extern "C"`, takes plain device pointers, element
 * counts and a HIP stream passed as `void*` (a hipStream_t; NULL = the legacy
 * default stream), never allocates user tensors, launches asynchronously on
 * that stream and returns an `int` status (OC_OK on success). A failed call
 * leaves a human-readable reason in oc_last_error() (thread-local).
 *
 * Layouts follow the reference's AutoGPTQ / RTN checkpoint formats:
 *   qweight  int32 [ceil(K/8), N]  8 nibbles per word, packed along K:
 *            code(k, n) = (qweight[k/8][n] >> (4*(k%8))) & 0xF
 *   qzeros   int32 [G, N/8]        8 nibbles per word, packed along N:
 *            zst(g, n) = (qzeros[g][n/8] >> (4*(n%8))) & 0xF
 *            V1 ("gptq")    zero = (zst + 1) & 0xF
 *            V2 ("gptq_v2") zero = zst
 *   scales   fp16/bf16 [G, N]
 *   RTN      uint8 [rows, ceil(K/2)]  byte j holds col 2j (low nibble) and
 *            col 2j+1 (high nibble); scales/zeros [rows, G] (G = 1: per row)
 *
 * Reference citations are relative to the onecompression-runtime source tree.
 */
#ifndef ONECOMP_HIP_H
#define ONECOMP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define OC_OK 0
#define OC_ERR_INVALID_ARGUMENT 1 /* bad pointer / dtype / flag            */
#define OC_ERR_SHAPE 2            /* shape or alignment contract violated  */
#define OC_ERR_UNSUPPORTED 3      /* valid but not implemented here        */
#define OC_ERR_WORKSPACE 4        /* workspace missing or too small        */
#define OC_ERR_HIP 5              /* a HIP runtime call failed             */

/* ---- element types ----------------------------------------------------- */
#define OC_DTYPE_F16 1
#define OC_DTYPE_BF16 2
#define OC_DTYPE_F32 3
#define OC_DTYPE_U8 4
#define OC_DTYPE_I32 5

/* ---- zero-point conventions -------------------------------------------- */
#define OC_ZERO_V1 1 /* stored zero-1, restored as (z+1)&0xF (format "gptq")  */
#define OC_ZERO_V2 2 /* stored zero as is (format "gptq_v2")                 */

/* ---- GEMM regime selection (oc_int4_gemm `regime`) ---------------------- */
#define OC_REGIME_AUTO 0
#define OC_REGIME_SPLITK 1 /* small-M MFMA kernel, K split over the waves (M <= 64) */
#define OC_REGIME_TILED 2  /* large-M LDS-tiled MFMA kernel                  */
#define OC_REGIME_DOT 3    /* decode kernel (M <= 2): VALU dot2, factored scales */

/* Human-readable name of a status code. */
const char *oc_status_string(int status);

/* Detail message of the last failed call on this thread ("" if none). */
const char *oc_last_error(void);

/* ABI version (major*10000 + minor*100 + patch). */
int oc_version(void);

/*
 * Host-only (no GPU needed): plan the physical row layout that turns any
 * GPTQ grouping into uniform groups of `group_rows` rows (a multiple of 32).
 *
 * Group g's input columns (k with g(k) == g, ascending k) occupy physical
 * rows [g*group_rows, g*group_rows + count_g); the remaining rows of the
 * slot are zero rows (kmap = -1). g(k) = g_idx[k] when g_idx != NULL
 * (act-order), else k / groupsize. This single re-layout covers
 *   - act-order g_idx (replaces the per-call `scales[g_idx]` gather of
 *     quant_utils.py:66-67 by a load-time row permutation),
 *   - odd group sizes < 32 (the reference's _repack_groups_to_32,
 *     layers/fused_int4_linear.py:94-124, and its activation remap at
 *     :370-376),
 *   - K not a multiple of the group size (K padding, :989-1045).
 * Outputs: kmap_out[K_phys] (activation column of each physical row, -1 for
 * a zero row), *k_phys_out, *group_rows_out, *num_groups_out, and
 * *identity_out = 1 when kmap is the identity (kmap[k] == k, K_phys == K),
 * in which case the GEMM may be called with kmap = NULL.
 * If kmap_out is NULL only the sizes are returned (query mode).
 */
int oc_int4_plan_groups(const int64_t *g_idx, int32_t K, int32_t groupsize,
                        int32_t *kmap_out, int64_t kmap_capacity,
                        int32_t *k_phys_out, int32_t *group_rows_out,
                        int32_t *num_groups_out, int32_t *identity_out);

/*
 * Device, load time: build the tiled layout ("tile16") every GEMM entry
 * point reads. Output features are cut into tiles of 16; within a tile the
 * 32-row K steps follow each other, and within a step the 16 columns' 4
 * packed words are adjacent (one 16-byte load = a whole 32-row group of one
 * column; a wave instruction reads 1 KB of consecutive bytes):
 *   qt  int32 [tiles][K_phys/32][16][4]   word (t, ks, c, w) = the codes of
 *        physical rows 32ks + 8w .. +7 of column 16t + c, where physical row
 *        k' holds input row kmap[k'] (zero code for -1; kmap NULL = identity
 *        with rows >= K zero)
 *   st  16-bit [tiles][G][16]            scale of (group, column 16t + c)
 *   zt  int32 [tiles][G][2]              8 zero points per word, stored as
 *        the zero itself (a v1 checkpoint's stored zero-1 is restored here)
 * tiles = ceil(N/16), G = K_phys / group_rows; columns past N are zero.
 * Inputs: qweight [ceil(K/8), N], scales [>= G, N], qzeros [>= G, N/8] in
 * the checkpoint formats (header comment). Replaces the load-time repacks of
 * layers/fused_int4_linear.py:76-124 (_pack_int4_weights,
 * _repack_groups_to_32) and the K padding at :1016-1045.
 */
int oc_int4_prepare(const int32_t *qweight, int32_t K, int32_t N,
                    const int32_t *kmap, int32_t K_phys, int32_t group_rows,
                    const void *scales, int32_t scale_dtype,
                    const int32_t *qzeros, int32_t zero_mode, int32_t *qt,
                    void *st, int32_t *zt, void *stream);

/*
 * Device, load time: the 8-bit counterpart of oc_int4_prepare (GPTQ wbits=8:
 * 4 codes per int32 word, mask 0xFF, quant_utils.py:21-22). Same arguments;
 * inputs qweight [ceil(K/4), N], qzeros [>= G, N/4] (v1 restores
 * (z + 1) & 0xFF); N % 4 == 0. Output layout ("tile16x8"):
 *   qt  int32 [tiles][K_phys/32][16][8]   word (t, ks, c, w) = the codes of
 *        physical rows 32ks + 4w .. +3 (byte i = row 4w + i) of column 16t + c
 *   st  16-bit [tiles][G][16]            as in the 4-bit layout
 *   zt  int32 [tiles][G][4]              4 zero bytes per word (columns
 *        16t + 4h .. +3), stored as the zero itself
 */
int oc_int8_prepare(const int32_t *qweight, int32_t K, int32_t N,
                    const int32_t *kmap, int32_t K_phys, int32_t group_rows,
                    const void *scales, int32_t scale_dtype,
                    const int32_t *qzeros, int32_t zero_mode, int32_t *qt,
                    void *st, int32_t *zt, void *stream);

/*
 * Device: fused 8-bit GPTQ dequant + GEMM over the oc_int8_prepare layout,
 * C = A' @ Wd + bias with Wd = RNE_a(f32(scale) * (code - zero)) exactly as
 * dequant_gptq_to_fp (quant_utils.py:50-69) and fp32 accumulation; the
 * fused counterpart of PackedGPTQLinear.forward for wbits = 8
 * (layers/packed_gptq_linear.py:66-74), which dequantizes the whole weight
 * per call. Arguments and workspace as oc_int4_gemm (one LDS-tiled MFMA
 * kernel at every M; K split over fp32 partials when the grid is small;
 * act-order rows gathered into the workspace). N % 4 == 0.
 */
int oc_int8_gemm(const void *a, int64_t lda, int32_t a_dtype, int32_t M,
                 int32_t K_logical, const int32_t *qt, const void *st,
                 int32_t scale_dtype, const int32_t *zt, int32_t N,
                 int32_t K_phys, int32_t group_rows, const int32_t *kmap,
                 const uint16_t *kinv, const void *bias, int32_t bias_dtype,
                 void *c, int64_t ldc, void *workspace, size_t workspace_bytes,
                 void *stream);

/* Workspace bytes oc_int8_gemm needs for this call shape (0 if none). */
size_t oc_int8_gemm_workspace_bytes(int32_t M, int32_t N, int32_t K_phys,
                                    int32_t group_rows, int32_t has_kmap);

/* Device: the 8-bit counterpart of oc_int4_export (qweight
 * [ceil(out_rows/4), N], qzeros [out_groups, N/4]; v1 stores zero - 1 mod 256). */
int oc_int8_export(const int32_t *qt, const void *st, const int32_t *zt,
                   int32_t N, int32_t K_phys, int32_t group_rows,
                   const int32_t *row_src, int32_t out_rows,
                   int32_t out_groups, int32_t zero_mode, int32_t *qweight,
                   void *scales, int32_t *qzeros, void *stream);

/* Device: the 8-bit counterpart of oc_int4_dequant_tiled. */
int oc_int8_dequant_tiled(const int32_t *qt, const void *st,
                          int32_t scale_dtype, const int32_t *zt,
                          const int32_t *kmap, int32_t N, int32_t K_phys,
                          int32_t group_rows, int32_t K_logical, void *out,
                          int32_t out_dtype, void *stream);

/*
 * Device, checkpoint export (state_dict): the inverse of oc_int4_prepare.
 * Writes the layer back in the checkpoint formats of the header comment, in
 * the buffer layout the reference's modules register:
 *   qweight int32 [ceil(out_rows/8), N]: code row k = physical row
 *           row_src[k] (NULL: k itself); -1 or a row past K_phys is a zero code
 *   scales  16-bit [out_groups, N] (st's dtype), qzeros int32 [out_groups, N/8];
 *           groups past K_phys/group_rows get zero scales and zero words
 *   zero_mode OC_ZERO_V1 stores zero - 1 (mod 16), OC_ZERO_V2 the zero.
 * The reference layouts this reproduces: FusedInt4Linear's K padded to a
 * multiple of 256 with zero rows/scales/zeros (layers/fused_int4_linear.py:
 * 989-1005, :1016-1045; identity rows, out_rows = padded K);
 * FusedInt4LinearPaddedGroups' 32-row group slots (:800-803, the physical
 * order itself); PackedGPTQLinear's and FusedInt4LinearAnyGroup's verbatim
 * checkpoint tensors (packed_gptq_linear.py:57-59, fused_int4_linear.py:
 * 660-662; row_src = the physical row of each input row).
 */
int oc_int4_export(const int32_t *qt, const void *st, const int32_t *zt,
                   int32_t N, int32_t K_phys, int32_t group_rows,
                   const int32_t *row_src, int32_t out_rows,
                   int32_t out_groups, int32_t zero_mode, int32_t *qweight,
                   void *scales, int32_t *qzeros, void *stream);

/*
 * Device, test/inspection and the fp32-activation path: dense out[N, K_logical]
 * (original K order) from the tiled layout, each value RNE_out(s * (code - zero))
 * exactly as quant_utils.dequant_gptq_to_fp (quant_utils.py:50-69).
 */
int oc_int4_dequant_tiled(const int32_t *qt, const void *st,
                          int32_t scale_dtype, const int32_t *zt,
                          const int32_t *kmap, int32_t N, int32_t K_phys,
                          int32_t group_rows, int32_t K_logical, void *out,
                          int32_t out_dtype, void *stream);

/*
 * Device: unpack int32-packed `wbits` codes along dim 0,
 *   out[r, c] = (packed[r / (32/wbits), c] >> (wbits * (r % (32/wbits)))) & mask
 * for r < num_rows; out is int32 [num_rows, cols]. Replaces
 * quant_utils._unpack_rows (quant_utils.py:12-28). wbits in {2, 4, 8}.
 */
int oc_unpack_rows(const int32_t *packed, int32_t packed_rows, int32_t cols,
                   int32_t wbits, int32_t num_rows, int32_t *out, void *stream);

/*
 * Device, test/inspection only: dequantize a GPTQ layer to out [N, K]
 * (row n = output feature), bit-exact with quant_utils.dequant_gptq_to_fp
 * (quant_utils.py:50-69):
 *   out[n, k] = RNE_out( f32(scales[g(k), n]) * f32(code(k, n) - zero(g(k), n)) )
 * g(k) = g_idx[k] (int32, device) or k / groupsize when g_idx == NULL.
 * wbits in {4, 8} (8-bit: 4 codes per word, mask 0xFF). scale_dtype in
 * {F16, BF16, F32}; out_dtype in {F16, BF16, F32}.
 */
int oc_int4_dequant(const int32_t *qweight, const void *scales,
                    int32_t scale_dtype, const int32_t *qzeros,
                    int32_t zero_mode, const int32_t *g_idx, int32_t groupsize,
                    int32_t wbits, int32_t K, int32_t N, void *out,
                    int32_t out_dtype, void *stream);

/*
 * Device: fused int4 dequant + GEMM, C[M, N] = A' @ Wd + bias, where
 *   A'[m, k'] = kmap ? (kmap[k'] >= 0 ? A[m, kmap[k']] : 0) : A[m, k'],
 *   Wd[k', n] = RNE_a( f32(scale) * (code(k', n) - zero) )   (see oc_int4_prepare)
 * computed with fp32 accumulation and rounded once to a_dtype on store
 * (bias added in fp32). The small-batch kernels (M <= 16 on the balanced
 * ranges, the whole-tile decode kernel) evaluate the same sum with the
 * scale and zero factored out of each 32-row group: there each weight enters
 * as the exact fp32 product s * (code - zero), not rounded to a_dtype first,
 * so results differ from dequantize-then-multiply by at most that rounding
 * per weight (and are identical for a one-hot row without bias). Replaces the
 * Triton launches of layers/fused_int4_linear.py:1194-1208
 * (FusedInt4Linear.forward), :504-532 (fused_int4_gemm) and :904-919
 * (FusedInt4LinearPaddedGroups.forward), and the act-order packed path
 * layers/packed_gptq_linear.py:66-74.
 *   a        [M, K_logical] (row stride lda elements, lda % 8 == 0, 16-byte
 *            aligned), a_dtype in {F16, BF16}
 *   qt/st/zt tiled weights from oc_int4_prepare (scale_dtype F16 or BF16)
 *   kmap     NULL or int32 [K_phys] (device, 16-byte aligned)
 *   kinv     NULL or uint16 [K_logical] (device, 16-byte aligned), the
 *            inverse of kmap: kinv[kmap[k']] = k'. Activations are permuted
 *            through it (coalesced) when given; without it the decode regime
 *            gathers through kmap (its split-item kernel).
 *   bias     NULL or [N] of bias_dtype in {F16, BF16, F32}
 *   c        [M, N] (row stride ldc elements) of a_dtype
 * Constraints: N % 8 == 0, K_phys % 32 == 0, group_rows % 32 == 0,
 * K_phys % group_rows == 0; without kmap K_logical == K_phys; the layer's
 * packed words below 2 GiB (N * K_phys / 2 bytes, 16 columns per tile).
 * The workspace (>= oc_int4_gemm_workspace_bytes, 256-byte aligned) starts
 * with a 512 KB counter area (small-batch calls, M <= 16: arrival counters
 * and the 64-bit cells through which two workgroups sharing an output tile
 * exchange their partial sums), then holds gathered activations (kmap with
 * M > 2, unless the batch's rows are staged in LDS) and fp32
 * split-K partials (large M with few output tiles, or a decode call whose K
 * is split over workgroups). The counter area must hold zeros the
 * first time a workspace is used (e.g. allocate it zero-filled) and every
 * call leaves it zero again; the rest may hold anything. Calls that overlap
 * in time must not share a workspace. `regime`: OC_REGIME_*.
 */
int oc_int4_gemm(const void *a, int64_t lda, int32_t a_dtype, int32_t M,
                 int32_t K_logical, const int32_t *qt, const void *st,
                 int32_t scale_dtype, const int32_t *zt, int32_t N,
                 int32_t K_phys, int32_t group_rows, const int32_t *kmap,
                 const uint16_t *kinv, const void *bias, int32_t bias_dtype,
                 void *c, int64_t ldc,
                 void *workspace, size_t workspace_bytes, int32_t regime,
                 void *stream);

/*
 * Device: oc_int4_gemm without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the reference. Same arguments, math
 * and regimes as oc_int4_gemm; the scratch it needs (counter area, gathered
 * activations, split-K partials) comes from a static device array of the
 * library, oc_int4_gemm_noalloc_scratch_bytes() bytes (32 MiB) per device,
 * held by every GPU the library runs on until the process ends. Calls whose
 * scratch need exceeds it return OC_ERR_WORKSPACE. The call allocates nothing
 * (no hipMalloc / hipFree / allocating library routine). Every call on one
 * GPU shares that GPU's array: calls that overlap in time on one GPU (two
 * streams, or a graph replay beside an eager call) race and must not be
 * issued. The first call on a device looks the array up and clears its
 * counter area with a kernel on `stream`.
 */
int oc_int4_gemm_noalloc(const void *a, int64_t lda, int32_t a_dtype,
                         int32_t M, int32_t K_logical, const int32_t *qt,
                         const void *st, int32_t scale_dtype,
                         const int32_t *zt, int32_t N, int32_t K_phys,
                         int32_t group_rows, const int32_t *kmap,
                         const uint16_t *kinv, const void *bias,
                         int32_t bias_dtype, void *c, int64_t ldc,
                         int32_t regime, void *stream);

/* Bytes of the static scratch behind oc_int4_gemm_noalloc (per device). */
size_t oc_int4_gemm_noalloc_scratch_bytes(void);

/* Workspace bytes oc_int4_gemm needs for this call shape (0 if none). */
size_t oc_int4_gemm_workspace_bytes(int32_t M, int32_t N, int32_t K_phys,
                                    int32_t group_rows, int32_t has_kmap,
                                    int32_t regime);

/*
 * Device, test/inspection only: RTN uint8-nibble dequant, bit-exact with
 * quant_utils.dequant_extra_u8_to_weight (quant_utils.py:72-103): every
 * operation is rounded to out_dtype (RNE), as torch does for 16-bit math:
 *   w = code; zq = RNE(zero); sq = RNE(scale); d = RNE(w - zq); out = RNE(d * sq)
 * qweight_u8 [rows, row_bytes] with row_bytes >= ceil(K/2); scales/zeros
 * [rows, G] with K % G == 0 (G == 1: per row). out [rows, K].
 * scale_dtype in {F16, BF16, F32}; zero_dtype in {F16, BF16, F32, U8, I32}.
 */
int oc_rtn_dequant(const uint8_t *qweight_u8, int32_t rows, int32_t row_bytes,
                   const void *scales, int32_t scale_dtype, const void *zeros,
                   int32_t zero_dtype, int32_t G, int32_t K, void *out,
                   int32_t out_dtype, void *stream);

/*
 * Device: fused RTN linear, C[M, N] = X @ Wrtn^T + bias, with Wrtn the
 * per-op-rounded dequant above in x_dtype, fp32 accumulation, one rounding
 * on store. Replaces PackedRTNLinear.forward (layers/packed_linear.py:53-56).
 * x [M, K] (row stride ldx), x_dtype in {F16, BF16}; qweight_u8 [N, row_bytes];
 * scales/zeros [N, G]; bias NULL or [N] (rounded to x_dtype first, like
 * `bias.to(x.dtype)` at packed_linear.py:55); c [M, N] (row stride ldc).
 */
int oc_rtn_linear(const void *x, int64_t ldx, int32_t x_dtype, int32_t M,
                  int32_t K, const uint8_t *qweight_u8, int32_t row_bytes,
                  const void *scales, int32_t scale_dtype, const void *zeros,
                  int32_t zero_dtype, int32_t G, int32_t N, const void *bias,
                  int32_t bias_dtype, void *c, int64_t ldc, void *stream);

/*
 * Device: packed RTN embedding lookup, out[t, :] = dequant(row ids[t]) in
 * out_dtype. Replaces PackedEmbedding.forward (layers/packed_linear.py:93-104);
 * the reference's output dtype rule (scales' dtype, fp16 for non-float
 * scales, :98) is applied by the caller through out_dtype. ids are int64;
 * an id outside [0, V) yields a zero row and sets the device flag
 * `bad_id_flag` (int32, may be NULL) to 1.
 */
int oc_rtn_embedding(const int64_t *ids, int64_t T, const uint8_t *qweight_u8,
                     int64_t V, int32_t row_bytes, const void *scales,
                     int32_t scale_dtype, const void *zeros, int32_t zero_dtype,
                     int32_t G, int32_t D, void *out, int32_t out_dtype,
                     int32_t *bad_id_flag, void *stream);

/*
 * DeepSeek-V4 QEP packed layers (layers/dsv4_packed_linear.py:22-102):
 *   qweight uint8 [N, row_bytes]: per = 8 / wbits codes per byte along the
 *           in-dim, code(n, k) = (qweight[n][k / per] >> (wbits * (k % per)))
 *           & (2^wbits - 1) (int4: the RTN nibble order; int2: 4 per byte)
 *   scales / zeros of scale_dtype / zero_dtype in {F16, BF16, F32}, element
 *           (n, g) at n * sz_stride_n + g * sz_stride_g (either orientation of
 *           the reference's [G, N] / [N, G]); g = k / groupsize, or one per
 *           row when groupsize <= 0
 *   Wd[n, k] = RNE_out( fp32( fp32(code - zero) * scale ) )   (two fp32 ops)
 */
/* Device: dense out [N, K] (bit-exact with dequant_dsv4_packed; wbits 2, 4, 8). */
int oc_dsv4_dequant(const uint8_t *qweight, int32_t N, int32_t row_bytes,
                    int32_t wbits, int32_t K, const void *scales,
                    int32_t scale_dtype, const void *zeros, int32_t zero_dtype,
                    int32_t groupsize, int64_t sz_stride_n, int64_t sz_stride_g,
                    void *out, int32_t out_dtype, void *stream);

/*
 * Device: fused DSV4 dequant + GEMM, C[M, N] = X @ Wd^T + bias, Wd rounded to
 * x_dtype as above (the reference dequantizes to x.dtype and calls F.linear,
 * dsv4_packed_linear.py:94-98), fp32 accumulation, bias rounded to x_dtype by
 * the caller. wbits in {2, 4}; K % 32 == 0; groupsize % 8 == 0 or <= 0;
 * row_bytes >= K / per and a multiple of 4 (int4) or 2 (int2). LDS-tiled
 * MFMA kernel at every M, K split over fp32 partials in the workspace
 * (>= oc_dsv4_gemm_workspace_bytes, zero-filled counter area first) when
 * the grid is small. The weights may sit in a staging buffer filled by an
 * asynchronous host-to-device copy on another stream (expert offload).
 */
int oc_dsv4_gemm(const void *x, int64_t ldx, int32_t x_dtype, int32_t M,
                 int32_t K, const uint8_t *qweight, int32_t row_bytes,
                 int32_t wbits, const void *scales, int32_t scale_dtype,
                 const void *zeros, int32_t zero_dtype, int32_t groupsize,
                 int64_t sz_stride_n, int64_t sz_stride_g, int32_t N,
                 const void *bias, int32_t bias_dtype, void *c, int64_t ldc,
                 void *workspace, size_t workspace_bytes, void *stream);

/* Workspace bytes oc_dsv4_gemm needs for this call shape (0 if none). */
size_t oc_dsv4_gemm_workspace_bytes(int32_t M, int32_t N, int32_t K);

/*
 * Packed int4 convolutions (layers/packed_conv.py:123-222), groups = 1, RTN
 * weights as the reference's quantize_conv_weight writes them (:63-90):
 * qweight uint8 [rows, row_bytes] nibbles (RTN order), scales / zeros
 * [rows, G], dequant per op in x_dtype as dequant_extra_u8_to_weight.
 *
 * Conv1d: weight rows = C_out, columns ci * kernel_size + kk;
 *   y[b, o, t] = bias[o] + sum_{ci, kk} Wd[o, ci * k + kk] *
 *                x[b, ci, t * stride + kk * dilation - pad_left] (0 outside [0, L))
 * x [B, C_in, L], y [B, C_out, T_out], fp32 accumulation, one rounding. The
 * caller folds the reference's pad (_conv1d_pad, :93-105) and the conv's own
 * padding into pad_left and T_out. Needs C_in * kernel_size % 32 == 0 and
 * (C_in * kernel_size / G) % 8 == 0. Workspace >= oc_rtn_conv1d_workspace_bytes
 * (a bounded chunk of im2col rows and fp32 partials).
 */
int oc_rtn_conv1d(const void *x, int32_t x_dtype, int32_t B, int32_t C_in,
                  int32_t L, const uint8_t *qweight, int32_t row_bytes,
                  const void *scales, int32_t scale_dtype, const void *zeros,
                  int32_t zero_dtype, int32_t G, int32_t C_out,
                  int32_t kernel_size, int32_t stride, int32_t dilation,
                  int32_t pad_left, int32_t T_out, const void *bias,
                  int32_t bias_dtype, void *y, void *workspace,
                  size_t workspace_bytes, void *stream);
size_t oc_rtn_conv1d_workspace_bytes(int32_t B, int32_t C_in, int32_t C_out,
                                     int32_t kernel_size, int32_t T_out);

/*
 * Load time, Conv1d (no reference counterpart: the reference dequantizes the
 * weight for every call, layers/packed_conv.py:196-222): the RTN rows
 * [N = C_out, row_bytes] (K = C_in * kernel_size codes each) re-laid for the
 * large-M GEMM kernel, tiles of 16 output columns:
 *   qt[((t * KS + ks) * 16 + c) * 4 + w]  codes of K rows 32 ks + 8 w .. + 7
 *                                         of column 16 t + c (KS = K / 32)
 *   sz[(t * G + g) * 16 + c]              scale | zero << 16 (16-bit values)
 * with ceil(N / 16) tiles (columns past N zero): qt holds tiles * KS * 64 and
 * sz tiles * G * 16 32-bit words (qt 16-byte aligned). fast[0] / fast[1]
 * (device int32[2]) become 1 when every group's (scale, zero) allows the
 * exact single-rounding dequant for bf16 / fp16 activations (an integral
 * zero of magnitude <= 240 and a scale in (2^-100, 2^100) after rounding to
 * that dtype), else 0. Needs K % 32 == 0, K / G % 32 == 0, row_bytes % 4 == 0,
 * scales and zeros [N, G] of one 16-bit dtype.
 */
int oc_rtn_tile_prepare(const uint8_t *qweight, int32_t N, int32_t row_bytes,
                        int32_t K, const void *scales, const void *zeros,
                        int32_t dtype, int32_t G, int32_t *qt, uint32_t *sz,
                        int32_t *fast, void *stream);

/*
 * oc_rtn_conv1d with the tile layout of the same weight (oc_rtn_tile_prepare;
 * the reference interface is the one oc_rtn_conv1d cites). Chunks of 1024 or
 * more output rows run on the large-M kernel when tiles_fast (the flag
 * oc_rtn_tile_prepare reported for x_dtype) is nonzero, the group size is 32
 * times a power of two, C_out % 8 == 0 and scales / zeros share a 16-bit
 * dtype; other chunks, or qt / sz NULL, as oc_rtn_conv1d. Same workspace.
 * Results match oc_rtn_conv1d to fp32 summation order (one-hot products
 * bit-identical).
 */
int oc_rtn_conv1d_prepared(const void *x, int32_t x_dtype, int32_t B,
                           int32_t C_in, int32_t L, const uint8_t *qweight,
                           int32_t row_bytes, const void *scales,
                           int32_t scale_dtype, const void *zeros,
                           int32_t zero_dtype, int32_t G, const int32_t *qt,
                           const uint32_t *sz, int32_t tiles_fast,
                           int32_t C_out, int32_t kernel_size, int32_t stride,
                           int32_t dilation, int32_t pad_left, int32_t T_out,
                           const void *bias, int32_t bias_dtype, void *y,
                           void *workspace, size_t workspace_bytes,
                           void *stream);

/*
 * Load time, ConvTranspose1d: the stored weight [rows = C_in, cols =
 * C_out * kernel_size] (quant groups along cols) re-laid as
 * qweight_t [cols, rows / 2] (RTN nibbles along C_in) and scales_t /
 * zeros_t [G, rows] (16-bit); rows even.
 */
int oc_rtn_transpose_prepare(const uint8_t *qweight, int32_t rows,
                             int32_t row_bytes, int32_t cols,
                             const void *scales, const void *zeros, int32_t G,
                             uint8_t *qweight_t, void *scales_t, void *zeros_t,
                             void *stream);

/*
 * ConvTranspose1d over the re-laid weight:
 *   y[b, o, t] = bias[o] + sum_{ci, kk, j: j * stride + kk * dilation - padding = t}
 *                x[b, ci, j] * Wd[ci, o * k + kk]
 * x [B, C_in, L_in], y [B, C_out, L_out] (L_out as torch's conv_transpose1d,
 * output_padding included; the reference's unpad is a slice of y). Needs
 * C_in % 32 == 0; scales_t / zeros_t of one 16-bit scale_dtype. Workspace >=
 * oc_rtn_conv_transpose1d_workspace_bytes.
 */
int oc_rtn_conv_transpose1d(const void *x, int32_t x_dtype, int32_t B,
                            int32_t C_in, int32_t L_in,
                            const uint8_t *qweight_t, const void *scales_t,
                            const void *zeros_t, int32_t scale_dtype, int32_t G,
                            int32_t C_out, int32_t kernel_size, int32_t stride,
                            int32_t dilation, int32_t padding, int32_t L_out,
                            const void *bias, int32_t bias_dtype, void *y,
                            void *workspace, size_t workspace_bytes,
                            void *stream);
size_t oc_rtn_conv_transpose1d_workspace_bytes(int32_t B, int32_t C_in,
                                               int32_t L_in, int32_t C_out,
                                               int32_t kernel_size,
                                               int32_t L_out);

/*
 * Load time, ConvTranspose1d (no reference counterpart, as
 * oc_rtn_tile_prepare): the stored weight [K = C_in rows, N = C_out *
 * kernel_size cols] (quant groups along the cols) re-laid for the large-M
 * kernel with activations of x_dtype:
 *   qt[((t * KS + ks) * 16 + c) * 4 + w]  codes of rows 32 ks + 8 w .. + 7 of
 *                                         column 16 t + c (KS = K / 32)
 *   szt[t * K + row]                      sq | zq << 16: the row's scale and
 *                                         zero for the tile's column group,
 *                                         rounded to x_dtype (its bits)
 * with ceil(N / 16) tiles (past N zero): tiles * KS * 64 and tiles * K 32-bit
 * words, both 16-byte aligned. fast[0] (device int32) becomes 1 when every
 * (scale, zero) allows the exact single-rounding dequant for x_dtype, else 0.
 * Needs K % 32 == 0, N / G a multiple of 16, scales / zeros [K, G] of one
 * 16-bit dtype.
 */
int oc_rtn_tile_prepare_t(const uint8_t *qweight, int32_t K,
                          int32_t row_bytes, int32_t N, const void *scales,
                          const void *zeros, int32_t scale_dtype, int32_t G,
                          int32_t x_dtype, int32_t *qt, uint32_t *szt,
                          int32_t *fast, void *stream);

/*
 * oc_rtn_conv_transpose1d with the transposed tile layout of the same weight
 * (oc_rtn_tile_prepare_t for x_dtype; the reference interface is the one
 * oc_rtn_conv_transpose1d cites). Chunks of 1024 or more input positions run
 * their GEMM on the large-M kernel when tiles_fast (the flag the prepare step
 * reported) is nonzero and C_out * kernel_size % 8 == 0; other chunks, or qt
 * / szt NULL, as oc_rtn_conv_transpose1d. Same workspace. Results match it to
 * fp32 summation order (one-hot inputs bit-identical).
 */
int oc_rtn_conv_transpose1d_prepared(const void *x, int32_t x_dtype, int32_t B,
                                     int32_t C_in, int32_t L_in,
                                     const uint8_t *qweight_t,
                                     const void *scales_t, const void *zeros_t,
                                     int32_t scale_dtype, int32_t G,
                                     const int32_t *qt, const uint32_t *szt,
                                     int32_t tiles_fast, int32_t C_out,
                                     int32_t kernel_size, int32_t stride,
                                     int32_t dilation, int32_t padding,
                                     int32_t L_out, const void *bias,
                                     int32_t bias_dtype, void *y,
                                     void *workspace, size_t workspace_bytes,
                                     void *stream);

/*
 * Device: MoE routing prologue (no reference counterpart: the reference has
 * no grouped GEMM; its MoE path loops over experts, layers/dsv4_packed_linear.py:95-98).
 * Stable counting sort of the T*topk (token, slot) pairs by expert id:
 *   expert_offsets[E+1] (exclusive prefix of per-expert counts),
 *   sorted_pairs[T*topk] = pair index p = t*topk + j, grouped by expert,
 *   ascending p within an expert. Ids outside [0, E) are dropped (not
 *   counted). topk_ids is int64 [T, topk]. Single workgroup; T*topk <= 65536,
 *   E <= 1024.
 */
int oc_moe_route(const int64_t *topk_ids, int32_t T, int32_t topk, int32_t E,
                 int32_t *expert_offsets, int32_t *sorted_pairs, void *stream);

/*
 * Device: grouped int4 GEMM over E experts (no reference counterpart; see
 * oc_moe_route). For every routed pair p = t*topk + j of expert e:
 *   Y[p, :] = X[t, :] @ Wd_e        (fp32 accumulation, rounded to x_dtype)
 * x [T, K] (row stride ldx) in {F16, BF16}; per-expert tiled weights
 * (oc_int4_prepare of each expert, identity kmap) stacked on a leading E
 * axis: qt [E][N/16][K/32][16][4], st [E][N/16][G][16], zt [E][N/16][G][2];
 * y [T*topk, N] (row stride ldy). K % 32 == 0, group_rows % 32 == 0,
 * N % 64 == 0.
 */
int oc_int4_moe_gemm(const void *x, int64_t ldx, int32_t x_dtype, int32_t T,
                     int32_t topk, int32_t K, const int32_t *qt,
                     const void *st, int32_t scale_dtype, const int32_t *zt,
                     int32_t group_rows, int32_t E, int32_t N,
                     const int32_t *expert_offsets, const int32_t *sorted_pairs,
                     void *y, int64_t ldy, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ONECOMP_HIP_H */
