/*
 * mtl_decode.h -- C ABI of the batch-1 decode-step kernels around the int4 GEMV
 * (MI355X / gfx950).  Same conventions as mtl_gptq.h: 0 = MTL_OK, negative =
 * MTL_ERR_*, raw device pointers, bf16 as 16-bit patterns, a hipStream_t, no
 * allocation or host synchronisation, capturable into a hipGraph.
 *
 * The decode position is read from device memory (`pos`, int64), so one
 * captured step serves every cache length (the reference captures one graph
 * per length: moss_tts_lite/fast_native.py:369-386).
 */
#ifndef MTL_DECODE_H
#define MTL_DECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * RMSNorm over rows, op for op as the reference's Qwen3RMSNorm
 * (moss_tts_lite/model.py:34-40): out = bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))
 * with fp32 statistics.  x, w, out bf16; x [rows, n], w [n]; out may alias x.
 */
int mtl_rmsnorm(const void* x, const void* w, void* out, int64_t rows, int64_t n,
                float eps, void* stream);

/*
 * Embedding lookup and sum (moss_tts_lite/model.py:156-161, fast.py:123-128):
 * out = bf16(...bf16(T0[ids[0]] + T1[ids[1]]) + ...), each table bf16 [vocab_i, hidden].
 *   ids     int64 [n_tables] (device), 1 <= n_tables <= 64
 *   tables  device array of n_tables table base pointers
 *   vocabs  device array of n_tables row counts (ids outside [0, vocab) read as 0)
 */
int mtl_embed_sum(const int64_t* ids, int32_t n_tables, const void* const* tables,
                  const int64_t* vocabs, int64_t hidden, void* out, void* stream);

/*
 * mtl_embed_sum that also prepares the first decoder layer's RMSNorm-staged GEMV (the
 * input RMSNorm of moss_tts_lite/model.py:169 on the summed embedding): the same out, plus
 *   slots   float [hidden / 16]: sum of squares of out's columns 16b .. 16b+15, bit for bit
 *           as mtl_residual_add forms it with part = NULL
 *   h_ord   bf16 [hidden] or NULL: h_ord[scatter[d]] = out[d] (scatter NULL: h_ord[d])
 * hidden % 256 == 0 and hidden <= 16384, else MTL_ERR_SHAPE.
 */
int mtl_embed_sum_stats(const int64_t* ids, int32_t n_tables, const void* const* tables,
                        const int64_t* vocabs, int64_t hidden, void* out,
                        const int32_t* scatter, void* h_ord, float* slots, void* stream);

/*
 * Per-head q/k RMSNorm, RoPE and KV-cache write for one decode position
 * (moss_tts_lite/fast.py:134-147, model.py:175-185).
 *   qkv      bf16 [(n_heads + 2*n_kv_heads) * head_dim] = q | k | v projections
 *   q_norm_w, k_norm_w  bf16 [head_dim]
 *   cos_tab, sin_tab    bf16 [max_seq, head_dim] (model.py:115-124)
 *   pos      int64 device scalar; positions outside [0, max_seq) write nothing
 *   q_out    bf16 [n_heads * head_dim] (normed, rotated)
 *   k_cache, v_cache  bf16 [n_kv_heads, max_seq, head_dim] of this layer
 * head_dim must be 128.
 */
int mtl_qk_norm_rope_kv(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                        const void* cos_tab, const void* sin_tab, const int64_t* pos,
                        void* q_out, void* k_cache, void* v_cache, int32_t n_heads,
                        int32_t n_kv_heads, int32_t head_dim, int64_t max_seq, float eps,
                        void* stream);

/*
 * Same, with the projection given as the fp32 split-K partials of the q|k|v GEMV
 * ([splits, (n_heads + 2*n_kv_heads)*head_dim], from mtl_w4_gemm_partials): each
 * projection value is bf16(sum over splits, in split order) before the norm.
 */
int mtl_qk_norm_rope_kv_partials(const float* partials, int32_t splits, const void* q_norm_w,
                                 const void* k_norm_w, const void* cos_tab, const void* sin_tab,
                                 const int64_t* pos, void* q_out, void* k_cache, void* v_cache,
                                 int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                 int64_t max_seq, float eps, void* stream);

/*
 * Residual add + RMSNorm of the fused step (moss_tts_lite/fast.py:168-169 then
 * model.py:34-40).  With partials (fp32 [splits, n] of the o or down GEMV):
 * h_out = bf16(bf16(sum of partials) + resid) (h_out may alias resid); without:
 * h = resid.  Then x = RMSNorm(h, w), written as x_out[j] = x[gather[j]] (the act-order
 * input order of the next int4 GEMV) or x_out = x when gather is NULL.  n % 4 == 0,
 * n <= 16384.
 */
int mtl_residual_rmsnorm(const float* partials, int32_t splits, const void* resid, void* h_out,
                         const void* w, void* x_out, const int32_t* gather, int64_t n, float eps,
                         void* stream);

/*
 * GQA decode attention over cache positions [0, pos] (the reference's SDPA call at
 * moss_tts_lite/fast.py:149-162, exact length pos + 1): one launch, split over the
 * sequence in chunks of at most 64 positions (up to 64 chunks), fp32 softmax, chunk
 * results merged in chunk order by the last workgroup of each kv head.
 *   q    bf16 [n_heads * head_dim];  out bf16 [n_heads * head_dim]
 *   out_index  NULL, or int32 [n_heads * head_dim]: value i is written to
 *              out[out_index[i]] (the act-order input order of the o projection)
 *   scale  softmax scale (1/sqrt(head_dim) in the reference)
 *   workspace  mtl_decode_attention_workspace_bytes(n_heads, head_dim) bytes, 16-byte
 *              aligned, ZERO-FILLED before its first use (every launch leaves its
 *              counters zero again); one stream at a time.
 * head_dim must be 128; n_heads % n_kv_heads == 0, n_heads / n_kv_heads <= 8,
 * n_kv_heads <= 127.
 * pos < 0 writes nothing; pos >= max_seq attends over [0, max_seq).
 */
int64_t mtl_decode_attention_workspace_bytes(int32_t n_heads, int32_t head_dim);

/*
 * Hand-off of the chunk partials between the attention's workgroups (no counterpart in
 * the reference: an implementation choice of mtl_decode_attention and
 * mtl_decode_attention_fused, process-wide, read at each launch).
 *   1 (default)  XCD-local: the chunks of one kv head run on one XCD (n_kv_heads a
 *                multiple of 8, workgroups dispatched to the XCDs in turn by linear id),
 *                so partials and the arrival count stay in that XCD's L2.  A launch that
 *                finds a kv head's chunks on more than one XCD adds 1 to the uint32 at
 *                byte 1016 of the workspace (the placement word, zero when it held).
 *   0            agent-scope stores, release count and acquire fence (any placement).
 * Returns MTL_ERR_INVALID_ARG for other values.
 */
int mtl_decode_attention_set_handoff(int32_t local);
int mtl_decode_attention(const void* q, const void* k_cache, const void* v_cache,
                         const int64_t* pos, void* out, const int32_t* out_index, int32_t n_heads,
                         int32_t n_kv_heads, int32_t head_dim, int64_t max_seq, float scale,
                         void* workspace, int64_t ws_bytes, void* stream);

/*
 * bf16 output head with greedy selection: logits[n] = bf16(sum_k W[n,k] x[k])
 * (moss_tts_lite/fast.py:180, F.linear with a bf16 weight [N, K]) and
 * token_out[0] = argmax(logits) (first maximum; NaN counts as the maximum).
 * Either output may be NULL.  K % 8 == 0.
 */
int64_t mtl_head_workspace_bytes(int64_t N);
int mtl_bf16_gemv_argmax(const void* x, const void* w, int64_t N, int64_t K, void* logits,
                         int64_t* token_out, void* workspace, int64_t ws_bytes, void* stream);

/*
 * Residual add of the norm-staged step (moss_tts_lite/fast.py:168-169): with partials
 * (fp32 [splits, n] of the o or down GEMV) h = bf16(bf16(sum of partials) + h) in place;
 * without, h is only read.  slots[b] receives the sum of squares of h over columns
 * 16b .. 16b+15 (consumed by mtl_w4_gemm_norm_partials / mtl_bf16_gemv_argmax_norm,
 * which apply the RMSNorm of model.py:34-40).  h_ord (optional) receives h scattered
 * into the next int4 GEMV's act-order input order: h_ord[scatter[i]] = h[i] (scatter
 * NULL: copy).  n % 4 == 0, n <= 16384.
 */
int mtl_residual_add(const float* partials, int32_t splits, void* h, const int32_t* scatter,
                     void* h_ord, float* slots, int64_t n, void* stream);

/*
 * mtl_qk_norm_rope_kv_partials and mtl_decode_attention in one pass: q/k RMSNorm,
 * RoPE and the KV write of position pos are done inside the attention workgroups
 * from the q|k|v split-K partials (fast.py:134-162).  Same workspace and limits.
 * The q/k/v projections of position pos are not written anywhere except the cache.
 */
int mtl_decode_attention_fused(const float* qkv_partials, int32_t splits, const void* q_norm_w,
                               const void* k_norm_w, const void* cos_tab, const void* sin_tab,
                               void* k_cache, void* v_cache, const int64_t* pos, void* out,
                               const int32_t* out_index, int32_t n_heads, int32_t n_kv_heads,
                               int32_t head_dim, int64_t max_seq, float scale, float eps,
                               void* workspace, int64_t ws_bytes, void* stream);

/*
 * mtl_bf16_gemv_argmax on x = RMSNorm(h, norm_w) (the final norm, model.py:34-40 and
 * fast.py:179-180), with h's sums of squares per 16 columns in slots (16-byte aligned).
 */
int mtl_bf16_gemv_argmax_norm(const void* h, const void* norm_w, const float* slots, float eps,
                              const void* w, int64_t N, int64_t K, void* logits,
                              int64_t* token_out, void* workspace, int64_t ws_bytes,
                              void* stream);

/*
 * mtl_bf16_gemv_argmax_norm followed by mtl_advance_position, the end of a captured
 * greedy decode step (moss_tts_lite/fast.py:179-180 and the next position), with the
 * position advanced by the argmax's own last launch: one launch fewer.  token_out and
 * pos are required (else MTL_ERR_INVALID_ARG).
 */
int mtl_bf16_gemv_argmax_norm_advance(const void* h, const void* norm_w, const float* slots,
                                      float eps, const void* w, int64_t N, int64_t K,
                                      void* logits, int64_t* token_out, int64_t* pos,
                                      void* workspace, int64_t ws_bytes, void* stream);

/*
 * bf16 GEMV without selection: out[n] = bf16(sum_k W[n,k] x[k]) for W bf16 [N, K]
 * (F.linear with a bf16 weight: the text, audio and 2-way heads of
 * moss_tts_lite/fast.py:174-194, and bf16-kept projections, gptq.py:689-697).  When
 * pad_period > 0, rows with n % pad_period == pad_index are written as -inf (the audio
 * heads' pad code, fast.py:181-182).  K % 8 == 0, K <= 12288.
 */
int mtl_bf16_gemv(const void* x, const void* w, int64_t N, int64_t K, void* out,
                  int64_t pad_period, int64_t pad_index, void* stream);

/*
 * A linear kept in bf16 inside the decode step (the reference's F.linear on a kept
 * projection, moss_tts_lite/gptq.py:689-693, e.g. v_proj in the shipped GPTQ presets,
 * export.py:59-72): out[n] = bf16(sum_k x[k] W[n, k]) stored as fp32, where
 * x = RMSNorm(h) = bf16(norm_w * bf16(h * rsqrt(sum(slots)/K + eps))) is formed while
 * staging (slots: the sums of squares of h per 16 columns).  The fp32 values are bf16
 * numbers, for consumers that read fp32 partials (one split).  W bf16 [N, K] row-major;
 * K % 8 == 0, K <= 12288; h, norm_w, slots, W 16-byte aligned.
 */
int mtl_bf16_gemv_norm(const void* h, const void* norm_w, const float* slots, float eps,
                       const void* w, int64_t N, int64_t K, float* out, void* stream);

/* pos[0] += 1 on the device (ends a captured decode step). */
int mtl_advance_position(int64_t* pos, void* stream);

/*
 * SwiGLU of a layer whose up_proj stays bf16 (the w2 preset keeps it on some layers,
 * moss_tts_lite/export.py:66-70) while gate_proj is int4:
 * act[i] = bf16(silu(bf16 gate[i]) * bf16 up[i]) (moss_tts_lite/fast.py:170-171), from the
 * two projections' fp32 outputs.  n elements (any rows x columns, contiguous).
 */
int mtl_silu_mul_f32(const float* gate, const float* up, void* act, int64_t n, void* stream);

/* ---- Prefill: every prompt row in one launch (moss_tts_lite/fast.py:210-270) ---- */

/*
 * Embedding sum of `rows` rows (fast.py:210-216): ids int64 [rows, n_tables] (device),
 * tables/vocabs as mtl_embed_sum; out bf16 [rows, hidden].
 */
int mtl_embed_rows(const int64_t* ids, int64_t rows, int32_t n_tables, const void* const* tables,
                   const int64_t* vocabs, int64_t hidden, void* out, void* stream);

/*
 * RMSNorm of each row (model.py:34-40, as mtl_rmsnorm) written in the act-order input
 * order of the next int4 GEMM: out[r][j] = norm(x[r])[gather[j]] (gather NULL: no
 * permutation).  x, w, out bf16; rows ldx / ldo elements apart (multiples of 8, 16-byte
 * aligned); n % 8 == 0, n <= 16384.  In place only with ldx == ldo.
 */
int mtl_rmsnorm_gather(const void* x, int64_t ldx, const void* w, const int32_t* gather,
                       void* out, int64_t ldo, int64_t rows, int64_t n, float eps, void* stream);

/*
 * The residual add of a K-split o or down GEMM and the next RMSNorm + gather in one launch
 * (fast.py:230-250 on prompt rows): h[r] = bf16(bf16(sum over the splits of partials, in
 * split order) + h[r]) in place (partials fp32 [splits][rows][n], from
 * mtl_w4_gemm_prefill_partials), then out[r] as mtl_rmsnorm_gather of the new h.  The
 * same bits as mtl_w4_gemm_prefill's residual launch followed by mtl_rmsnorm_gather.
 * splits 1..8; out must not be h; MTL_ERR_WORKSPACE when partials_bytes < splits * rows *
 * n * 4.  sums: NULL, or out staged as mtl_rmsnorm_gather_staged stages it.
 */
int mtl_residual_rmsnorm_gather(const float* partials, int32_t splits, int64_t partials_bytes,
                                void* h, int64_t ldh, const void* w, const int32_t* gather,
                                void* out, int64_t ldo, float* sums, int64_t rows, int64_t n,
                                float eps, void* stream);

/*
 * mtl_rmsnorm_gather with its output staged for mtl_w4_gemm_prefill_staged: each 8-channel
 * item of out in pair order (x0,x4),(x1,x5),(x2,x6),(x3,x7), and sums fp32 [rows][n/32] the
 * sums of out's 32-channel groups, as the GEMM's own staging forms them.  n % 32 == 0;
 * gather 16-byte aligned.  mtl_residual_rmsnorm_gather stages the same way when its sums
 * is not NULL.  No counterpart in the reference (its linears take the normed rows).
 */
int mtl_rmsnorm_gather_staged(const void* x, int64_t ldx, const void* w, const int32_t* gather,
                              void* out, int64_t ldo, float* sums, int64_t rows, int64_t n,
                              float eps, void* stream);

/*
 * q/k RMSNorm, RoPE and KV-cache write for `rows` rows at positions pos0 .. pos0+rows-1
 * (fast.py:226-237), the arithmetic of mtl_qk_norm_rope_kv per row.
 *   qkv    bf16 [rows, ldq], each row q | k | v ((n_heads + 2 n_kv_heads) * 128)
 *   q_out  bf16 [rows, n_heads * 128]
 * head_dim must be 128; pos0 + rows <= max_seq.
 */
int mtl_qk_norm_rope_kv_rows(const void* qkv, int64_t ldq, int64_t rows, int64_t pos0,
                             const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                             const void* sin_tab, void* q_out, void* k_cache, void* v_cache,
                             int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                             int64_t max_seq, float eps, void* stream);

/*
 * mtl_qk_norm_rope_kv_rows on the q|k|v GEMM's K-split partial sums instead of its bf16
 * output (mtl_w4_gemm_prefill_partials): the heads whose 128 columns lie below part_cols
 * take bf16(sum of the splits in split order) from partials fp32 [splits][rows][part_cols],
 * the same bits as the GEMM's split-sum launch writes; the heads past part_cols (a
 * bf16-kept v_proj's, gptq.py:689-693) read qkv bf16 [rows, ldq] (NULL when part_cols
 * covers every head).  part_cols a multiple of 128; splits 1..8; MTL_ERR_WORKSPACE when
 * partials_bytes < splits * rows * part_cols * 4.  The split sum, the q/k norms, RoPE and
 * the KV write in one launch (fast.py:220-237 on prompt rows).
 */
int mtl_qk_norm_rope_kv_rows_partials(const float* partials, int32_t splits,
                                      int64_t partials_bytes, int64_t part_cols,
                                      const void* qkv, int64_t ldq, int64_t rows, int64_t pos0,
                                      const void* q_norm_w, const void* k_norm_w,
                                      const void* cos_tab, const void* sin_tab, void* q_out,
                                      void* k_cache, void* v_cache, int32_t n_heads,
                                      int32_t n_kv_heads, int32_t head_dim, int64_t max_seq,
                                      float eps, void* stream);

/*
 * Causal GQA attention of `rows` query rows at positions pos0 + r over cache positions
 * [0, pos0 + r] (fast.py:238-242: SDPA, is_causal), scale as given (1/sqrt(head_dim) in
 * the reference).  Scores and the value sum on MFMA (bf16 operands, fp32 accumulation),
 * online softmax in fp32.
 *   q    bf16 [rows, n_heads * 128] (normed, rotated: mtl_qk_norm_rope_kv_rows)
 *   out  bf16 [rows, ldo]; value c of a row goes to column out_index[c] (NULL: c)
 * head_dim 128, n_heads / n_kv_heads <= 8, pos0 + rows <= max_seq.
 */
int mtl_prefill_attention(const void* q, const void* k_cache, const void* v_cache, int64_t rows,
                          int64_t pos0, void* out, int64_t ldo, const int32_t* out_index,
                          int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int64_t max_seq,
                          float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MTL_DECODE_H */
