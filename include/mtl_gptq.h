/*
 * mtl_gptq.h -- C ABI of the MI355X (gfx950) int4 GPTQ decode hot path.
 *
 * Library: moss-tts-lite_amd/libmtl_hip.so (hipcc --offload-arch=gfx950).
 *
 * Conventions shared by every entry point
 *   - Return 0 (MTL_OK) on success, a negative MTL_ERR_* code otherwise; no
 *     exception or abort crosses the ABI.  mtl_status_string() names a code.
 *   - All tensor arguments are raw DEVICE pointers to contiguous row-major
 *     memory owned by the caller; sizes are element counts.  bf16 and fp16
 *     values are passed as their 16-bit patterns.
 *   - `stream` is a hipStream_t (NULL = the null stream).  Launch paths do not
 *     allocate, synchronise or read device memory from the host, so every
 *     launch is capturable into a hipGraph.
 *   - Entry points are stateless and reentrant, except mtl_gptq_gemm_noalloc, whose
 *     calls on one GPU share a library-owned array.  A workspace belongs to one
 *     stream at a time: two launches that share a workspace must be ordered.
 *
 * Weight layouts.  AutoGPTQ: `qweight` int32 [K/8, N]; the 4-bit code of input channel
 * k = 8*i + j of output column n is bits [4j, 4j+4) of qweight[i*N + n] (low nibble
 * first).  The reference's contract (mtl_int4pack_*): the strip layout of that qweight
 * (mtl_w4_strip): 1 KB block (s * K/128 + b) holds columns 16s .. 16s+15 over input
 * channels 128b .. 128b+127, word j of its 16-byte word l the qweight word (row
 * 16b + 4j + l/16, column 16s + l%16).  A column strip is one contiguous K*8-byte run, so
 * the N*K/8 words, shaped as torch's [N/8, K/(16*T), 32, T/2], concatenate along dim 0
 * exactly as a concatenation of the weights along N.
 */
#ifndef MTL_GPTQ_H
#define MTL_GPTQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MTL_OK = 0,
  MTL_ERR_INVALID_ARG = -1,   /* null pointer, bad enum value            */
  MTL_ERR_SHAPE = -2,         /* M/K/N out of range or not divisible      */
  MTL_ERR_GROUP = -3,         /* group size not in {32, 64, 128, 256}     */
  MTL_ERR_ALIGN = -4,         /* pointer not 16-byte aligned              */
  MTL_ERR_WORKSPACE = -5,     /* workspace missing or too small           */
  MTL_ERR_LAUNCH = -6,        /* HIP launch error                         */
  MTL_ERR_UNSUPPORTED = -7    /* valid request the library does not serve */
};

/* Output element type of the GEMM entry points. */
enum { MTL_OUT_BF16 = 0, MTL_OUT_F32 = 1 };

/* Fused epilogues of mtl_w4_gemm_fused. */
enum {
  MTL_EPI_NONE = 0,       /* y = acc (bf16 or f32 per out_dtype)                       */
  MTL_EPI_RESIDUAL = 1,   /* y = bf16(bf16(acc) + resid)        (fast.py:168,170)      */
  MTL_EPI_SILU_MUL = 2    /* y[j] = bf16(silu(bf16 gate_j) * bf16 up_j); columns come
                             interleaved in blocks of 32 (gate|up) (fast.py:170-171)  */
};

/* Weight layout of the decode-step GEMV entries (mtl_w4_gemm_partials,
 * mtl_w4_gemm_norm_partials, mtl_w4_gemm_residual). */
enum {
  MTL_LAYOUT_ROWS = 0,    /* qweight int32 [K/8, N] as everywhere else                  */
  MTL_LAYOUT_TILED = 1,   /* mtl_w4_tile output (M = 1, N % 64 == 0, no perm)           */
  MTL_LAYOUT_STRIP = 2,   /* mtl_w4_strip output (M = 1, N % 16 == 0, K % 256 == 0,
                             K <= 16384, no perm), with scales/qzeros in the strip order
                             of mtl_w4_strip_meta: full-K strip GEMV, no split-K       */
  MTL_LAYOUT_STRIP_QSZ = 3 /* the same strip-layout weights (mtl_w4_strip, or the output of
                             mtl_int4pack_convert / mtl_int4pack_from_torch_tiles) with the
                             reference's metadata: `scales` is qsz bf16 [K/g, N, 2]
                             (w = (q - 8) * scale + zero), `qzeros` and zero_offset unused */
};

/* OR'ed into the xsplits argument of mtl_w4_gemm_residual (strip layouts): each split of
 * xpart holds the gate partials in its first K floats and the up partials in the next K,
 * instead of the 32-column gate|up interleave (a bf16-kept up_proj's output beside its
 * int4 gate's). */
enum { MTL_XPART_HALVES = 1 << 30 };

/* Metadata format of mtl_w4_gemm_fused. */
enum {
  MTL_META_GPTQ = 0,      /* scales fp16 [K/g,N] + qzeros int32 [K/g,N/8]; w=(q-z)*s  */
  MTL_META_QSZ = 1        /* qsz bf16 [K/g,N,2] = (scale, zero); w=(q-8)*scale+zero   */
};

const char* mtl_status_string(int status);
int mtl_abi_version(void);

/* Bytes of workspace a GEMM of this shape needs: a 16 KB tile-counter region
 * followed by fp32 split-K partial tiles.  mtl_gptq_gemm and mtl_w4_gemm_fused sum
 * their partials in a second launch and read no counter, so their workspace needs no
 * clearing; the entries that count workgroups (mtl_w4_gemm_residual and its _geom form)
 * need the counters zero before first use (mtl_workspace_init zero-fills), and every launch
 * leaves them zero. */
int64_t mtl_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int32_t group_size);
int mtl_workspace_init(void* workspace, int64_t ws_bytes, void* stream);

/*
 * AutoGPTQ-layout GEMM, y[M,N] = x[M,K] @ dequant(W)[K,N], fp32 accumulation.
 * Replaces the int4 GEMM the GPTQ linear dispatches to
 * (reference: torch._weight_int4pack_mm via kernel_linear,
 *  moss_tts_lite/gptq.py:577-585, 689-697).
 *   x        bf16 [M, K], 1 <= M <= 16
 *   qweight  int32 [K/8, N]  (group-sorted rows when perm != NULL)
 *   qzeros   int32 [K/g, N/8], nibble z; effective zero = z + zero_offset
 *   scales   fp16 [K/g, N]
 *   perm     NULL (no act-order), or int32 [K] from mtl_gptq_actorder_prepare:
 *            the kernel reads x[:, perm[k]] for sorted channel k
 *   y        bf16 or f32 [M, N] (out_dtype)
 * K % group_size == 0, group_size in {32,64,128,256}, N % 8 == 0.
 */
int mtl_gptq_gemm(const void* x, int64_t M, int64_t K,
                  const int32_t* qweight, const int32_t* qzeros, const void* scales,
                  const int32_t* perm, int64_t N, int32_t group_size,
                  int32_t zero_offset, void* y, int32_t out_dtype,
                  void* workspace, int64_t ws_bytes, void* stream);

/*
 * mtl_gptq_gemm without a workspace argument, and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under graph capture, tight serving loops).  The split-K workspace is a
 * library-owned static device array of MTL_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends; the first call on a device looks up its address (no stream operation, so
 * a first call under graph capture records only the GEMM's own launches).  Nothing in the
 * array needs clearing: the GEMM reads only partials the same call wrote.  Every call on
 * one GPU shares that array: calls that overlap on one GPU race and must be ordered by the
 * caller.  Arguments and results as mtl_gptq_gemm;
 * MTL_ERR_WORKSPACE when mtl_gemm_workspace_bytes(M, K, N, group_size) exceeds the
 * array (16 MiB: the decode shapes q|k|v 4096x6144, o 4096x4096, gate|up 4096x24576 and
 * down 12288x4096 fit at every M <= 16; gate|up at M = 16 needs 12 MiB).
 */
#define MTL_NOALLOC_SCRATCH_BYTES (16ll << 20)
int mtl_gptq_gemm_noalloc(const void* x, int64_t M, int64_t K,
                          const int32_t* qweight, const int32_t* qzeros, const void* scales,
                          const int32_t* perm, int64_t N, int32_t group_size,
                          int32_t zero_offset, void* y, int32_t out_dtype, void* stream);

/*
 * Act-order preparation: from an AutoGPTQ qweight whose input channels are
 * grouped by an arbitrary g_idx (desc_act=True checkpoints), write the
 * group-contiguous copy qweight_sorted[K/8, N] and the gather index perm[K]
 * (stable argsort of g_idx).  Every group must own exactly group_size
 * channels; otherwise MTL_ERR_GROUP.  `scratch` needs mtl_actorder_scratch_bytes(K).
 * This is the load-time step the GPTQ linear module runs once per layer.
 */
int64_t mtl_actorder_scratch_bytes(int64_t K);
int mtl_gptq_actorder_prepare(const int32_t* qweight, const int32_t* g_idx,
                              int64_t K, int64_t N, int32_t group_size,
                              int32_t* qweight_sorted, int32_t* perm,
                              void* scratch, int64_t scratch_bytes, void* stream);

/*
 * Reference-contract GEMM: y[M,N] = x[M,K] @ W^T with
 * W[n,k] = (q-8)*qsz[k/g,n,0] + qsz[k/g,n,1] (bf16 pair widened to fp32), fp32 sums.
 * Replaces torch._weight_int4pack_mm(x, packed, g, qsz) at
 * moss_tts_lite/fast.py:118, gptq.py:582, fast_native.py:169.
 *   x       bf16 [M, K], any M >= 1
 *   packed  strip layout from mtl_int4pack_convert or mtl_int4pack_from_torch_tiles
 *           (N*K/8 words; NOT torch's tiled bytes)
 *   qsz     bf16 [K/g, N, 2], read in place
 *   y       bf16 [M, N], 8-byte aligned
 *   workspace  NULL, or mtl_int4pack_mm_workspace_bytes(M, K, N) bytes: lets a launch
 *           with M > 1 split K over workgroups (results then differ by fp32 rounding)
 * M = 1 runs the full-K strip GEMV (K <= 16384); 2 <= M <= 16 the skinny strip GEMM
 * (mtl_w4_gemm_strip_rows_ex), more rows the prompt-length GEMM (N % 128 == 0; otherwise
 * the skinny GEMM 16 rows at a time).  K % 256 == 0, K % g == 0,
 * N % 16 == 0 (torch asks N % 8 only).
 */
int64_t mtl_int4pack_mm_workspace_bytes(int64_t M, int64_t K, int64_t N);
int mtl_int4pack_mm(const void* x, int64_t M, int64_t K, const int32_t* packed,
                    int32_t group_size, const void* qsz, int64_t N, void* y,
                    void* workspace, int64_t ws_bytes, void* stream);

/*
 * Reference-contract packer: the reference's nibble pre-pack uint8 [N, K/2]
 * (byte = q[n,2i]<<4 | q[n,2i+1], moss_tts_lite/fast.py:98, gptq.py:76) ->
 * packed: the strip layout, N*K/8 int32 words.  Replaces
 * torch.ops.aten._convert_weight_to_int4pack (fast.py:97, gptq.py:75); inner_k_tiles is
 * accepted for signature parity and must be 2, 4 or 8 (it does not change this layout).
 * K % 256 == 0, N % 16 == 0.
 */
int mtl_int4pack_convert(const uint8_t* prepacked, int64_t N, int64_t K,
                         int32_t inner_k_tiles, int32_t* packed, void* stream);

/*
 * torch's tiled int4 tensor -> packed, the strip layout of mtl_int4pack_convert.
 * Ingests the `.q` records of the reference's standalone export
 * (moss_tts_lite/export.py:324-334, read back at export.py:691-734 and handed to
 * torch._weight_int4pack_mm): the int32 [N/8, K/(16*T), 32, T/2] tensor that
 * torch.ops.aten._convert_weight_to_int4pack(pre, T) returns on a ROCm GPU.
 *   tiles          int32, N*K/8 words, 4-byte aligned
 *   inner_k_tiles  T in {2, 4, 8} (the export writes 8)
 *   N % 16 == 0, K % 256 == 0
 */
int mtl_int4pack_from_torch_tiles(const int32_t* tiles, int64_t N, int64_t K,
                                  int32_t inner_k_tiles, int32_t* packed, void* stream);

/*
 * Wave-contiguous copy of a qweight [K/8, N] for the decode-step GEMVs (load time):
 * 16-byte word l of 1 KB block ((s * N/64 + cg) * 16 + q) holds row 64s + 4q + l/16,
 * columns 64cg + 4(l%16) .. +3; rows past K/8 are zero.  Each GEMV wave then streams
 * 16 consecutive 1 KB blocks instead of 64 strided 256-byte pieces.  N % 64 == 0.
 * No reference counterpart (the reference's packed layout is torch's own).
 */
int64_t mtl_w4_tiled_bytes(int64_t K, int64_t N);
int mtl_w4_tile(const int32_t* qweight, int64_t K, int64_t N, int32_t* tiled, int64_t tiled_bytes,
                void* stream);

/*
 * Column-strip copy of a qweight [K/8, N] for the full-K strip GEMV (load time): 1 KB
 * block (s * K/128 + b) holds columns 16s .. 16s+15 over input channels 128b .. 128b+127,
 * its 16-byte word l the words (row 16b + 4j + l/16, column 16s + l%16), j = 0..3.  A
 * strip's blocks are consecutive, so one workgroup streams one contiguous K*8-byte run.
 * N % 16 == 0, K % 256 == 0; mtl_w4_strip_bytes returns 0 for other shapes.
 * No reference counterpart (the reference's packed layout is torch's own).
 */
int64_t mtl_w4_strip_bytes(int64_t K, int64_t N);
int mtl_w4_strip(const int32_t* qweight, int64_t K, int64_t N, int32_t* strip, int64_t strip_bytes,
                 void* stream);

/*
 * Strip-ordered copy of the group metadata for the strip GEMV (load time): for each
 * 16-column strip and each 128-channel block (block pair at g = 256), the MB = 128/g
 * scales of every column contiguously (fp16, MB = 1 at g = 256) and their zero nibbles
 * (column c's MB nibbles at nibble c*MB of the record).  A permutation of scales
 * [K/g, N] and of the qzeros nibbles: the outputs have the sizes of the inputs.  N % 16
 * == 0, K % 256 == 0; outputs 16-byte aligned.  No reference counterpart (the reference's
 * qsz tensor is torch's own layout).
 */
int mtl_w4_strip_meta(const void* scales, const int32_t* qzeros, int64_t K, int64_t N,
                      int32_t group_size, void* strip_scales, int32_t* strip_zeros,
                      void* stream);

/*
 * Skinny-batch int4 GEMM over the strip layout: y[M, N] = x[M, K] @ dequant(W), 1 <= M <= 16,
 * fp32 accumulation, no workspace.  Replaces torch._weight_int4pack_mm at M > 1, which the
 * reference's quantized prefill runs on every projection (moss_tts_lite/fast.py:218-270,
 * via _linear at fast.py:107-121).  A workgroup owns whole columns over all of K, so no
 * split-K partials are written; x of all M rows is staged once per workgroup.
 *   x             bf16 [M, K], rows ldx elements apart (16-byte aligned, ldx % 8 == 0)
 *   strip_weight  mtl_w4_strip output of qweight [K/8, N] (no act-order permutation: the
 *                 caller orders x's channels as the weight's rows)
 *   scales/qzeros as mtl_gptq_gemm; zero_offset as there
 *   y             [M, N] bf16 or f32 (out_dtype), rows ldy elements apart
 * K % 256 == 0, N % 16 == 0, N * K / 2 < 2^31; group_size 32, 64, 128 or 256.  x is staged
 * in LDS in phases of K sized for 16 rows (all of K at once up to K = 4096), the same at
 * every M, so a row's result does not depend on the rows launched with it.
 */
int mtl_w4_gemm_strip_rows(const void* x, int64_t M, int64_t ldx, int64_t K,
                           const int32_t* strip_weight, const void* scales,
                           const int32_t* qzeros, int64_t N, int32_t group_size,
                           int32_t zero_offset, void* y, int64_t ldy, int32_t out_dtype,
                           void* stream);

/*
 * mtl_w4_gemm_strip_rows for both metadata contracts and act-order inputs.  Replaces
 * torch._weight_int4pack_mm at 2 <= M <= 16 on the reference's own (packed, qsz) records
 * (moss_tts_lite/fast.py:107-121 at prompt rows, gptq.py:577-585), and serves the GPTQ
 * module's forward at M <= 16 with its act-order gather.
 *   perm         NULL, or int32 [K] (16-byte aligned): input row k of the weight multiplies
 *                x channel perm[k] (the act-order index of mtl_actorder_prepare; GPTQ
 *                metadata only)
 *   meta_format  MTL_META_GPTQ (meta = scales fp16 [K/g, N], qzeros int32 [K/g, N/8]) or
 *                MTL_META_QSZ (meta = qsz bf16 [K/g, N, 2], qzeros NULL, zero_offset 0)
 *   other arguments as mtl_w4_gemm_strip_rows; no K limit beyond N * K / 2 < 2^31 (K
 *   runs in phases whose x fits the LDS).
 */
int mtl_w4_gemm_strip_rows_ex(const void* x, int64_t M, int64_t ldx, int64_t K,
                              const int32_t* perm, const int32_t* strip_weight, const void* meta,
                              const int32_t* qzeros, int64_t N, int32_t group_size,
                              int32_t zero_offset, int32_t meta_format, void* y, int64_t ldy,
                              int32_t out_dtype, void* stream);

/*
 * One row on the full-K strip GEMV: y[N] = x[K] @ dequant(W) over a GPTQ linear's strip copy
 * (mtl_w4_strip of its group-sorted qweight, mtl_w4_strip_meta of its scales and zeros),
 * x in the checkpoint's channel order.  Serves the GPTQ module's forward at M = 1, the
 * product the reference's kernel_linear hands to torch._weight_int4pack_mm
 * (moss_tts_lite/gptq.py:577-585, 149-160); the reference's own (packed, qsz) records take
 * the same kernel through mtl_int4pack_mm.
 *   x             bf16 [K], 16-byte aligned
 *   perm          NULL, or uint16 [K] (16-byte aligned): a permutation of 0..K-1, row k of
 *                 the sorted weight multiplies x[perm[k]] (mtl_gptq_actorder_prepare's
 *                 index, narrowed); the launch copies x into LDS and gathers from there
 *                 while staging
 *   strip_weight, strip_scales, strip_zeros   as mtl_w4_gemm_partials with MTL_LAYOUT_STRIP
 *   y             [N] bf16 or f32 (out_dtype), 8- or 16-byte aligned
 * K % 256 == 0, K <= 16384 (K <= 12288 with perm), N % 16 == 0, N * K / 2 < 2^31; group
 * size 32, 64, 128 or 256.  The sums are the decode step's strip GEMV's (same launch shape).
 */
int mtl_w4_gemv_strip(const void* x, int64_t K, const uint16_t* perm,
                      const int32_t* strip_weight, const void* strip_scales,
                      const int32_t* strip_zeros, int64_t N, int32_t group_size,
                      int32_t zero_offset, int32_t out_dtype, void* y, void* stream);

/*
 * Prompt-length int4 GEMM over the strip layout: y[M, N] = x[M, K] @ dequant(W) for any
 * M >= 1, fp32 accumulation on MFMA, no workspace.  The reference's quantized prefill
 * runs every projection at M = prompt length through torch._weight_int4pack_mm
 * (moss_tts_lite/fast.py:218-270, via _linear at fast.py:107-121); this entry serves
 * those products.
 *   x             bf16 [M, K], rows ldx elements apart (16-byte aligned, ldx % 8 == 0), in
 *                 the weight's input (act-order sorted) channel order
 *   strip_weight  mtl_w4_strip output; strip_scales/strip_zeros the mtl_w4_strip_meta
 *                 outputs of the same linear; zero_offset as mtl_gptq_gemm
 *   epilogue      MTL_EPI_NONE: y [M, N] bf16 or f32 (out_dtype);
 *                 MTL_EPI_RESIDUAL: y is the bf16 residual stream [M, N], updated in place
 *                 as y = bf16(bf16(acc) + y) (fast.py:243, 246-248);
 *                 MTL_EPI_SILU_MUL: N columns interleaved gate|up in blocks of 32, y bf16
 *                 [M, N/2] = bf16(silu(bf16 gate) * bf16 up) (fast.py:247)
 *                 (the two epilogues need out_dtype MTL_OUT_BF16)
 *   ldy           row pitch of y in elements (>= N, or N/2 for MTL_EPI_SILU_MUL)
 *   workspace     NULL, or mtl_w4_gemm_prefill_workspace_bytes(M, K, N) bytes (16-byte
 *                 aligned, no initialisation): when the grid alone would leave CUs idle, K
 *                 is split over workgroups whose fp32 partial sums a second launch adds in
 *                 split order before the epilogue (results then differ from the one-pass
 *                 launch by fp32 rounding); a smaller or NULL workspace runs one pass.
 *                 The workspace size query returns 0 when no split is needed.
 * K % 256 == 0, N % 128 == 0, K % group_size == 0, group_size 32/64/128/256.
 */
int64_t mtl_w4_gemm_prefill_workspace_bytes(int64_t M, int64_t K, int64_t N);
int mtl_w4_gemm_prefill(const void* x, int64_t M, int64_t ldx, int64_t K,
                        const int32_t* strip_weight, const void* strip_scales,
                        const int32_t* strip_zeros, int64_t N, int32_t group_size,
                        int32_t zero_offset, int32_t epilogue, int32_t out_dtype, void* y,
                        int64_t ldy, float* workspace, int64_t ws_bytes, void* stream);
/* The same GEMM with the reference's metadata: qsz bf16 [K/g, N, 2] read in place,
 * W[n,k] = (q-8)*scale + zero (moss_tts_lite/gptq.py:87-97; the quantized prefill of
 * fast.py:218-270 runs its projections through torch._weight_int4pack_mm on such weights). */
int mtl_w4_gemm_prefill_qsz(const void* x, int64_t M, int64_t ldx, int64_t K,
                            const int32_t* strip_weight, const void* qsz, int64_t N,
                            int32_t group_size, int32_t epilogue, int32_t out_dtype, void* y,
                            int64_t ldy, float* workspace, int64_t ws_bytes, void* stream);

/*
 * The prompt-length GEMM's K-split partial sums only, for a caller that adds the splits
 * itself (mtl_qk_norm_rope_kv_rows_partials, mtl_residual_rmsnorm_gather: the split sum
 * and the next operation in one launch instead of the second launch and that one).
 * partials fp32 [splits][M][N] with splits = mtl_w4_gemm_prefill_partials_bytes(M, K, N) /
 * (M * N * 4) (the split count of mtl_w4_gemm_prefill's workspace launch, or 1: the sums
 * themselves); meta_format MTL_META_GPTQ (strip scales + zeros) or MTL_META_QSZ (qsz, zeros
 * unused); x_sums NULL (x plain) or x staged as mtl_w4_gemm_prefill_staged takes it.  Sums
 * equal those mtl_w4_gemm_prefill adds in its second launch.  No counterpart in the
 * reference: the split of its linears (fast.py:218-250) over two launches.
 */
int64_t mtl_w4_gemm_prefill_partials_bytes(int64_t M, int64_t K, int64_t N);
int mtl_w4_gemm_prefill_partials(const void* x, const float* x_sums, int64_t M, int64_t ldx,
                                 int64_t K, const int32_t* strip_weight, const void* meta,
                                 const int32_t* strip_zeros, int64_t N, int32_t group_size,
                                 int32_t zero_offset, int32_t meta_format, float* partials,
                                 int64_t partials_bytes, void* stream);

/*
 * mtl_w4_gemm_prefill (MTL_EPI_NONE or MTL_EPI_SILU_MUL) on x staged by its producer
 * (mtl_rmsnorm_gather_staged, mtl_residual_rmsnorm_gather with sums): x bf16 [M, ldx] with
 * each 8-channel item in pair order (x0,x4),(x1,x5),(x2,x6),(x3,x7), and x_sums fp32
 * [M][K/32] the sums of its 32-channel groups.  The GEMM then copies x into LDS instead of
 * reordering it and summing its groups in every workgroup; the results are the bits of
 * mtl_w4_gemm_prefill(_qsz) on the same x in natural order.  meta_format as
 * mtl_w4_gemm_prefill_partials.  No counterpart in the reference (fast.py:218-250 run the
 * linears on the normed rows).
 */
int mtl_w4_gemm_prefill_staged(const void* x, const float* x_sums, int64_t M, int64_t ldx,
                               int64_t K, const int32_t* strip_weight, const void* meta,
                               const int32_t* strip_zeros, int64_t N, int32_t group_size,
                               int32_t zero_offset, int32_t meta_format, int32_t epilogue,
                               int32_t out_dtype, void* y, int64_t ldy, float* workspace,
                               int64_t ws_bytes, void* stream);

/* Unpack qweight [K/8, N] -> codes uint8 [K, N] (index/parity checks). */
int mtl_unpack_codes(const int32_t* qweight, int64_t K, int64_t N, uint8_t* codes,
                     void* stream);

/* Dequantise to fp32 W[K, N] (AutoGPTQ meta; perm may be NULL) -- the exact
 * value the GEMM multiplies by; used by the bit-exact dequant checks. */
int mtl_gptq_dequant(const int32_t* qweight, const int32_t* qzeros, const void* scales,
                     int64_t K, int64_t N, int32_t group_size, int32_t zero_offset,
                     float* w_out, void* stream);
/* Same for the reference contract, from the strip layout of mtl_int4pack_convert:
 * fp32 W[K, N] = effective_weight(q, qsz).T (moss_tts_lite/gptq.py:87-97).
 * K % 256 == 0, N % 16 == 0. */
int mtl_qsz_dequant(const int32_t* packed, const void* qsz, int64_t K, int64_t N,
                    int32_t group_size, float* w_out, void* stream);

/*
 * General entry with a fused epilogue, used by the decode step.
 *   meta_format  MTL_META_GPTQ (meta0 = scales fp16, qzeros) or
 *                MTL_META_QSZ (meta0 = qsz bf16 [K/g,N,2], qzeros = NULL)
 *   epilogue     MTL_EPI_*; RESIDUAL reads resid[M,N] bf16 (may alias y);
 *                SILU_MUL writes y[M, N/2]
 */
int mtl_w4_gemm_fused(const void* x, int64_t M, int64_t K, const int32_t* qweight,
                      int32_t meta_format, const void* meta0, const int32_t* qzeros,
                      const int32_t* perm, int64_t N, int32_t group_size,
                      int32_t zero_offset, int32_t epilogue, const void* resid,
                      void* y, int32_t out_dtype, void* workspace, int64_t ws_bytes,
                      void* stream);

/*
 * Partials-only launch for fused consumers (the decode step): writes the fp32
 * split-K partial tiles partials[splits, M, N] (splits = mtl_w4_gemm_splits(K, N))
 * and nothing else; the consumer sums them in split order.  The activation comes
 * from x (bf16 [M, K], through perm when given) or, when xpart is set (M = 1),
 * from the fp32 partials of an interleaved gate|up GEMV ([xsplits, 2K], 32-column
 * gate|up blocks): x[j] = bf16(silu(bf16 gate_j) * bf16 up_j) (fast.py:170-171).
 * AutoGPTQ meta only.  layout: MTL_LAYOUT_ROWS, or MTL_LAYOUT_TILED with qweight from
 * mtl_w4_tile (M = 1, no perm), or MTL_LAYOUT_STRIP with qweight from mtl_w4_strip: each
 * workgroup then sums all of K itself and partials holds ONE split, the final fp32 sums
 * [N] (consumers pass xsplits = 1).
 */
int32_t mtl_w4_gemm_splits(int64_t K, int64_t N);
int mtl_w4_gemm_partials(const void* x, const float* xpart, int32_t xsplits, int64_t xpart_ld,
                         int64_t M, int64_t K, const int32_t* qweight, const void* scales,
                         const int32_t* qzeros, const int32_t* perm, int64_t N, int32_t group_size,
                         int32_t zero_offset, int32_t layout, float* partials,
                         int64_t partials_bytes, void* stream);

/*
 * Partials-only launch (M = 1) whose activation is RMSNorm(h) computed while staging
 * (moss_tts_lite/model.py:34-40): x[j] = bf16(w[j] * bf16(h[j] * r)),
 * r = rsqrt(sum(slots[0 .. ceil(K/16) - 1]) / K + eps).  h and w are bf16 [K], already
 * in this GEMV's act-order input order (w is the norm weight gathered by the same
 * perm); slots (16-byte aligned) are the sums of squares of h per 16 columns
 * (mtl_residual_add, mtl_w4_gemm_residual).  layout as mtl_w4_gemm_partials.
 */
int mtl_w4_gemm_norm_partials(const void* h, const void* w, const float* slots, float eps,
                              int64_t K, const int32_t* qweight, const void* scales,
                              const int32_t* qzeros, int64_t N, int32_t group_size,
                              int32_t zero_offset, int32_t layout, float* partials,
                              int64_t partials_bytes, void* stream);

/*
 * mtl_w4_gemm_norm_partials and mtl_bf16_gemv_norm(bh, bnorm_w, slots, eps, bweight, bn,
 * K, bout) over the same slots (the RMS of h) in one launch: the decode step's int4 q|k
 * GEMV beside its bf16-kept v_proj (the w2 preset keeps v_proj in bf16, gptq.py:689-697;
 * moss_tts_lite/model.py:169-173 forms q, k and v from the same normed h), or the int4
 * gate beside a kept up_proj.  With the strip layout, one strip per workgroup of 4 waves
 * and K <= 4096 the first N/16 workgroups run the GEMV and the rest the bf16 rows;
 * otherwise the two launches are issued.  Either way the results are the two entries'
 * bits.  bh, bnorm_w, bweight 16-byte aligned; bweight bf16 [bn, K]; bout fp32 [bn].
 */
int mtl_w4_gemm_norm_partials_bf16(const void* h, const void* w, const float* slots, float eps,
                                   int64_t K, const int32_t* qweight, const void* scales,
                                   const int32_t* qzeros, int64_t N, int32_t group_size,
                                   int32_t zero_offset, int32_t layout, float* partials,
                                   int64_t partials_bytes, const void* bh, const void* bnorm_w,
                                   const void* bweight, int64_t bn, float* bout, void* stream);

/*
 * M = 1 GEMV whose epilogue is the decode step's residual add (moss_tts_lite/fast.py:
 * 168-171): h[n] = bf16(bf16((x @ W)[n]) + h[n]) in place, h scattered into the next
 * RMSNorm-staged GEMV's act-order input order (h_ord[scatter[n]] = h[n]; scatter NULL:
 * h_ord[n] = h[n]; h_ord NULL: no copy), and slots[b] = sum of h^2 over columns
 * 16b .. 16b+15 (what mtl_w4_gemm_norm_partials and mtl_bf16_gemv_argmax_norm consume).
 * x is bf16 [K] or, with xpart, SiLU*up of an interleaved gate|up GEMV's partials (as
 * mtl_w4_gemm_partials), or with xsplits | MTL_XPART_HALVES (strip layouts only) of
 * [gate K | up K] splits.  Layouts ROWS and TILED reduce split-K inside the kernel and
 * need the workspace of mtl_gptq_gemm (counters zero before first use; every launch
 * leaves them zero); MTL_LAYOUT_STRIP needs none (workspace may be NULL).  N <= 16384.
 */
int mtl_w4_gemm_residual(const void* x, const float* xpart, int32_t xsplits, int64_t xpart_ld,
                         int64_t K, const int32_t* qweight, const void* scales,
                         const int32_t* qzeros, int64_t N, int32_t group_size, int32_t zero_offset,
                         int32_t layout, void* h, const int32_t* scatter, void* h_ord,
                         float* slots, void* workspace, int64_t ws_bytes, void* stream);

/*
 * M = 1 gate|up GEMV with RMSNorm staging (as mtl_w4_gemm_norm_partials) whose epilogue is
 * the SwiGLU product of moss_tts_lite/fast.py:170-171: act[j] = bf16(silu(bf16 g_j) *
 * bf16 u_j), where the N fused columns come in 64-column blocks of 32 gate | 32 up
 * (act has N/2 entries, 8-byte aligned).  MTL_LAYOUT_STRIP only (N % 64 == 0,
 * K % 256 == 0, K <= 8192: one workgroup holds 2 strips x 8 K slices of at most 8 blocks);
 * other layouts return MTL_ERR_UNSUPPORTED.
 */
int mtl_w4_gemm_norm_silu(const void* h, const void* w, const float* slots, float eps, int64_t K,
                          const int32_t* qweight, const void* scales, const int32_t* qzeros,
                          int64_t N, int32_t group_size, int32_t zero_offset, int32_t layout,
                          void* act, void* stream);

/*
 * Launch geometry of the full-K strip GEMV (MTL_LAYOUT_STRIP, MTL_LAYOUT_STRIP_QSZ).  No
 * counterpart in the reference: the entries below are the four strip-layout GEMV entries
 * above with the launch shape given explicitly instead of chosen by the library, for
 * callers that sweep or pin launch shapes (benchmarks, tests).  Every field 0 (or a NULL
 * geometry) means automatic, which is what the entries without _geom use.  The arithmetic
 * per column is the same in every geometry up to the number of K slices whose sums are
 * added (strips_per_wg and blocks_per_wave fix it); the ring depth changes only when loads
 * are issued, so outputs equal the automatic ring's bit for bit.
 *   strips_per_wg    CT, 16-column strips per workgroup: 1, 2 or 4 for the RMSNorm-staged
 *                    store, 2 or 6 for the SiLU*up epilogue (gate|up strip pairs), 1 for
 *                    the others; qsz metadata (MTL_LAYOUT_STRIP_QSZ): automatic only
 *   blocks_per_wave  NB, 128-channel blocks per wave: 2, 4, 6, 8 or 16 with K/128 % NB == 0
 *                    and (K/128/NB) * CT waves per workgroup within the kernel's limit
 *   ring             blocks in flight per wave: 2 (NB = 2 or 8), 4 (NB = 4, 8 or 16),
 *                    8 (NB = 8 or 16, g >= 64), 16 (NB = 16, g >= 64), or NB = 6's own
 *   xcd_order        1: each XCD runs a contiguous range of strips (when the workgroup
 *                    count is a multiple of 8); -1: workgroup id order; 0: automatic (1)
 * A geometry that does not fit returns MTL_ERR_SHAPE (NB, CT) or MTL_ERR_UNSUPPORTED.
 */
typedef struct mtl_strip_geometry {
  int32_t strips_per_wg;
  int32_t blocks_per_wave;
  int32_t ring;
  int32_t xcd_order;
} mtl_strip_geometry;

int mtl_w4_gemm_partials_geom(const void* x, const float* xpart, int32_t xsplits,
                              int64_t xpart_ld, int64_t M, int64_t K, const int32_t* qweight,
                              const void* scales, const int32_t* qzeros, const int32_t* perm,
                              int64_t N, int32_t group_size, int32_t zero_offset, int32_t layout,
                              float* partials, int64_t partials_bytes,
                              const mtl_strip_geometry* geom, void* stream);
int mtl_w4_gemm_norm_partials_geom(const void* h, const void* w, const float* slots, float eps,
                                   int64_t K, const int32_t* qweight, const void* scales,
                                   const int32_t* qzeros, int64_t N, int32_t group_size,
                                   int32_t zero_offset, int32_t layout, float* partials,
                                   int64_t partials_bytes, const mtl_strip_geometry* geom,
                                   void* stream);
int mtl_w4_gemm_residual_geom(const void* x, const float* xpart, int32_t xsplits,
                              int64_t xpart_ld, int64_t K, const int32_t* qweight,
                              const void* scales, const int32_t* qzeros, int64_t N,
                              int32_t group_size, int32_t zero_offset, int32_t layout, void* h,
                              const int32_t* scatter, void* h_ord, float* slots, void* workspace,
                              int64_t ws_bytes, const mtl_strip_geometry* geom, void* stream);
int mtl_w4_gemm_norm_silu_geom(const void* h, const void* w, const float* slots, float eps,
                               int64_t K, const int32_t* qweight, const void* scales,
                               const int32_t* qzeros, int64_t N, int32_t group_size,
                               int32_t zero_offset, int32_t layout, void* act,
                               const mtl_strip_geometry* geom, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MTL_GPTQ_H */
