/*
 * sunshape_hip.h -- C ABI of libsunshape_hip.so, the MI355X (gfx950) HIP
 * implementation of SunShape's compressed-KV attention path.
 *
 * The reference (gauravsaini/sunshape-mlx) has no FFI: its boundary is a set
 * of Python launchers in kernels.py that take MLX arrays, run one Metal
 * dispatch synchronously and return an array (or None on failure).  Each
 * entry point below replaces one of those launchers (cited per function);
 * the Python package sunshape_mlx_amd binds them with ctypes.
 *
 * Conventions
 *  - Every pointer argument is a device pointer owned by the caller (torch
 *    tensors in the Python layer).  The library allocates no device memory.
 *  - Calls are asynchronous on the given stream (a hipStream_t passed as
 *    void*; NULL is the null stream).
 *  - Return value: SS_OK (0) or a negative SS_ERR_* code.  The text of the
 *    last error of the calling thread is returned by ss_last_error().
 *    Argument and shape checks happen on the host before any launch.
 *  - Stateless and reentrant, except that calls sharing one decode workspace
 *    must not overlap (the workspace holds the call's split partials), and
 *    calls of ss_decode_attn_il8_noalloc on one GPU share its static scratch
 *    and must not overlap either.
 *  - dtype codes: SS_F32, SS_F16, SS_BF16.
 */
#ifndef SUNSHAPE_HIP_H
#define SUNSHAPE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SS_OK 0
#define SS_ERR_INVALID (-1)     /* bad argument or shape */
#define SS_ERR_UNSUPPORTED (-2) /* valid but not implemented for this shape */
#define SS_ERR_HIP (-3)         /* HIP runtime error */
#define SS_ERR_WORKSPACE (-4)   /* workspace missing or too small */
#define SS_ERR_WAIT (-5)        /* a bounded in-kernel wait gave up (ss_decode_wait_failures) */

#define SS_F32 0
#define SS_F16 1
#define SS_BF16 2

/* Library version string, e.g. "sunshape_hip 0.1.0 gfx950". */
const char *ss_version(void);

/* Text of the last error raised on the calling thread ("" if none). */
const char *ss_last_error(void);

/*
 * Block-VQ encode (key or value quantisation) into uint8 indices.
 * Replaces block_vq_quantize_metal (reference kernels.py:1037-1082, kernel
 * body kernels.py:995-1027) and the permutation of codec.py:435-436.
 *
 * Tokens are addressed as (b, h, t) with b < n_b, h < n_h, t < n_t; element j
 * of token (b,h,t) is keys[b*k_sb + h*k_sh + t*k_st + j] (strides in
 * elements of keys_dtype).  perm (int32[head_dim], may be NULL) gathers the
 * key into codec space: kp[j] = key[perm[j]].  For every block the index of
 * the nearest centroid (squared L2, ties -> lowest index; distances within
 * 4e-6 relative of the best are re-resolved in float64) is written to
 * out[b*o_sb + h*o_sh + t*o_st + blk] (strides in bytes).  Writing at
 * o_st-strided rows of a cache buffer is the KV-append path.
 *   centroids: float32 [n_blocks][n_centroids][block_dim], n_centroids <= 256.
 */
int ss_encode_blockvq(const void *keys, int keys_dtype, int64_t n_b, int64_t n_h,
                      int64_t n_t, int64_t k_sb, int64_t k_sh, int64_t k_st,
                      int head_dim, const int32_t *perm, const float *centroids,
                      int n_blocks, int n_centroids, int block_dim, uint8_t *out,
                      int64_t o_sb, int64_t o_sh, int64_t o_st, void *stream);

/*
 * Codebook of the matrix-core encoder, prepared once per codebook (no
 * reference counterpart: block_vq_quantize_metal, kernels.py:1037-1082,
 * reads the float32 centroids on every call).  centroids float32
 * [n_blocks <= 16][n_centroids <= 256][8].  Per block b: a power-of-two scale
 * s_b bringing the largest |centroid element| into [8, 16) (0 when the
 * block holds a non-finite value), the MFMA operand of every 32-centroid
 * tile (fp16 s_b*C split into hi and lo, and the split (1 - 2^-15)|s_b C|^2),
 * the squared norms |s_b C|^2 and their maximum.  ss_encode_codebook_bytes
 * gives the size; prepared must be 16-byte aligned.
 */
size_t ss_encode_codebook_bytes(int n_blocks);
int ss_encode_codebook(const float *centroids, int n_blocks, int n_centroids, int block_dim,
                       void *prepared, void *stream);

/*
 * ss_encode_blockvq with the prepared codebook of the same centroids (same
 * arguments, same indices; replaces block_vq_quantize_metal, reference
 * kernels.py:1037-1082).  Bulk encodes (block_dim 8, n_blocks <= 16, more
 * than 4096 (token, block) pairs) rank the codebook on the matrix cores:
 * a lower bound of every squared distance from v_mfma_f32_32x32x16_f16,
 * accepted when its runner-up clears the float error bound, otherwise the
 * block is ranked exactly as ss_encode_blockvq does.  Other shapes run the
 * ss_encode_blockvq kernels; prepared may then be null.
 */
int ss_encode_blockvq_prepared(const void *keys, int keys_dtype, int64_t n_b, int64_t n_h,
                               int64_t n_t, int64_t k_sb, int64_t k_sh, int64_t k_st,
                               int head_dim, const int32_t *perm, const float *centroids,
                               int n_blocks, int n_centroids, int block_dim, uint8_t *out,
                               int64_t o_sb, int64_t o_sh, int64_t o_st, const void *prepared,
                               void *stream);

/*
 * Query x centroid table  lut[r][b][c] = sum_d q'[r][b*bd+d] * C[b][c][d]
 * with q'[r][j] = round_to(q_dtype, q[r][perm[j]] * scale).
 * Replaces precompute_query_centroid_dots (reference codec.py:553-573; the
 * einsum of attention.py:52-53).  q: [n_rows][head_dim] (row stride
 * q_row_stride elements); lut: float32 [n_rows][n_blocks][n_centroids].
 */
int ss_build_lut(const void *q, int q_dtype, int64_t n_rows, int64_t q_row_stride,
                 int head_dim, const int32_t *perm, float scale,
                 const float *centroids, int n_blocks, int n_centroids,
                 int block_dim, float *lut, void *stream);

/*
 * Score gather  scores[r][t] = sum_b lut[r][b][idx[t*idx_row_stride + b]].
 * Replaces block_vq_score_metal (reference kernels.py:87-116, kernel body
 * kernels.py:59-77).  idx: uint8, row stride in bytes; scores: float32
 * [n_rows][n_tok] (row stride out_row_stride elements).
 */
int ss_score_gather(const float *lut, int64_t n_rows, int n_blocks, int n_centroids,
                    const uint8_t *idx, int64_t n_tok, int64_t idx_row_stride,
                    float *scores, int64_t out_row_stride, void *stream);

/*
 * The same gather for every (batch, KV head) pair in one launch (the
 * reference loops over them with one dispatch each, attention.py:44-73,
 * 268-305): head (b, h) uses lut[b][h] [n_rows][n_blocks][n_centroids]
 * (float32, contiguous over all heads) and the indices of token t at
 * idx[b*idx_sb + h*idx_sh + t*idx_st] (bytes; a cache's [B][H][cap][NB]
 * buffer read up to n_tok), and writes scores[b][h] [n_rows][n_tok].
 */
int ss_score_gather_heads(const float *lut, int64_t n_rows, int n_blocks, int n_centroids,
                          const uint8_t *idx, int64_t n_b, int64_t n_h, int64_t idx_sb,
                          int64_t idx_sh, int64_t idx_st, int64_t n_tok, float *scores,
                          void *stream);

/*
 * Workspace bytes needed by ss_decode_attn_* for the given shape and split
 * count (n_splits <= 0 selects the library's choice for the current device);
 * 0 when a single split suffices.  With more than one split the split
 * workgroups write per-split softmax partials (m, l, acc) to the workspace.
 * ss_decode_attn_il8 and ss_decode_attn_grouped_il merge them inside their
 * kernel (the last split of each column to finish, counted in the
 * workspace's first 64 KiB); the other entry points merge with a second
 * launch on the stream.  A workspace must be
 * zero-filled once before its first use; every completed call leaves its
 * counter area zero again.
 */
size_t ss_decode_workspace_bytes(int64_t batch, int n_q_heads, int n_kv_heads,
                                 int64_t t_q, int head_dim, int64_t t_kv,
                                 int n_splits);

/*
 * Bounded-wait failures of the matrix-core fused decodes
 * (ss_decode_attn_il8, ss_decode_attn_grouped_il[_hybrid]) on the current
 * device.  Their waves hand tiles over through LDS flags and wait for each
 * other at compute-wave barriers; every such wait gives up after a bounded
 * number of sleeps, so a broken hand-off ends the kernel instead of hanging
 * it, and sets a bit in a sticky per-device word (1 compute barrier, 2 ring
 * slot, 4 ring tile).  The output of such a launch is invalid.  This call
 * synchronizes `stream`, stores the word in *flags (may be NULL), clears it
 * when `clear` is nonzero and returns SS_ERR_WAIT if it was nonzero, else
 * SS_OK.  No reference counterpart: the reference's Metal kernels
 * (kernels.py:142-446, 588-928) have no cross-wave hand-off.
 */
int ss_decode_wait_failures(void *stream, int clear, unsigned int *flags);

/*
 * Address (in *flag) of a word of pinned, host-mapped memory into which a
 * wait that gives up also stores its bits (the last give-up's bits), in any
 * process-wide launch; ss_decode_wait_failures folds it into its report and
 * clears it with the device word.  The host can poll it with a plain load
 * and no synchronisation: it is nonzero once a failed launch has finished
 * running, so a caller that checks it before each launch reports a failure
 * on a later call without waiting on any stream.  No reference counterpart.
 */
int ss_decode_wait_flag_host(unsigned int **flag);

/*
 * Test hook: the number of sleeps after which those waits give up, for
 * launches issued after this call (process-wide); a negative value restores
 * the default (2^20, about 0.03 s).  A small limit makes waits give up while
 * every wave still ends normally, which is how the failure report above is
 * tested.  No reference counterpart.
 */
int ss_debug_set_spin_limit(int limit);

/*
 * Read-ceiling kernel (measurement, no reference counterpart): streams
 * `bytes` (a multiple of 16) from `buf` with plain 16-byte non-temporal
 * loads over n_workgroups x 256 threads; `sink` receives at most one word.
 * bench.py times it over the bytes of a decode step to state the fastest a
 * single launch can read them on this device.
 */
int ss_stream_read(const void *buf, int64_t bytes, int n_workgroups, uint32_t *sink,
                   void *stream);

/* Split count the library would choose (n_splits <= 0 in the calls below). */
int ss_decode_default_splits(int64_t batch, int n_q_heads, int n_kv_heads,
                             int64_t t_q, int head_dim, int64_t t_kv);

/*
 * Fused GQA decode/prefill attention over block-VQ keys with dense values.
 * Replaces fused_attention_metal / fused_attention_causal_metal (reference
 * kernels.py:233-291, 388-446) driven per (b, kv head, q head) by
 * sunshape_sdpa (attention.py:199-305): one launch serves every query head of
 * every KV group.
 *   q       [batch][n_q_heads][t_q][head_dim] contiguous, q_dtype
 *           (query head hq reads KV head hq / (n_q_heads / n_kv_heads));
 *           the kernel forms round_to(q_dtype, q * scale), then q[perm].
 *   idx     uint8 [batch][n_kv_heads][cap][n_blocks] (first t_kv tokens used)
 *   values  [batch][n_kv_heads][cap][head_dim], v_dtype (SS_F16/SS_BF16/SS_F32)
 *   out     [batch][n_q_heads][t_q][head_dim], out_dtype
 *   causal  query row i (0 <= i < t_q) attends to keys t <= q_offset + i.
 * Softmax is accumulated in float32; rows with no admissible key output 0.
 */
int ss_decode_attn_dense(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                         int n_kv_heads, int64_t t_q, int head_dim, float scale,
                         const int32_t *perm, const float *centroids, int n_blocks,
                         int n_centroids, const uint8_t *idx, const void *values,
                         int v_dtype, int64_t cap, int64_t t_kv, int causal,
                         int64_t q_offset, void *out, int out_dtype, void *workspace,
                         size_t workspace_bytes, int n_splits, void *stream);

/*
 * Split count and workspace bytes a decode call of the given kind would use
 * (kind 0: ss_decode_attn_dense / ss_decode_attn_grouped, kind 1:
 * ss_decode_attn_il8 / ss_decode_attn_grouped_il).  Either output pointer may be NULL.
 */
int ss_decode_plan(int kind, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
                   int head_dim, int64_t t_kv, int n_splits, int *splits_out,
                   size_t *workspace_bytes_out);

/*
 * Codebook operand of ss_decode_attn_il8, prepared once per codebook (no
 * reference counterpart: the reference passes float32 centroids to every
 * fused_attention_metal call, kernels.py:233-291).  centroids float32
 * [n_blocks][n_centroids][8] is scaled by a power of two 2^-e (max |C| * 2^-e
 * < 2^14) and split into fp16 parts C' = hi + lo * 2^-11, stored in the
 * kernel's operand order: for 4-block group bg < n_blocks/4 and centroid
 * tile ct < ceil(n_centroids/16), tile (bg*ceil(n_centroids/16) + ct) holds
 * hi[64][8] then lo[64][8], row l being centroid ct*16 + l%16 of block
 * bg*4 + l/16 (zero past the last centroid); the float 2^e follows in a
 * 16-byte field, then |C|^2 (float32, unscaled) of every tile row in the
 * same order (the exact encode of ss_decode_step_il8 uses them).
 * n_blocks must be a multiple of 4.  ss_codebook_f16x2_bytes gives the
 * size; out must be 16-byte aligned.
 */
size_t ss_codebook_f16x2_bytes(int n_blocks, int n_centroids);
int ss_codebook_f16x2(const float *centroids, int n_blocks, int n_centroids, void *out,
                      void *stream);

/*
 * As ss_decode_attn_dense for fp16 values held in the cache's 8-token
 * interleaved layout: element (t, d) of a (batch, KV head) row lives at
 * values_il8[((b*n_kv_heads + h)*cap/8 + t/8)*head_dim*8 + d*8 + t%8]
 * (cap % 8 == 0), with the codebook prepared by ss_codebook_f16x2.  Both the
 * query x centroid LUT (split-fp16 v_mfma_f32_16x16x32_f16: exact fp16
 * products, fp32 accumulation) and P.V (v_mfma_f32_16x16x32_f16 with the
 * probabilities split into fp16 hi/lo parts) run on the matrix cores; four
 * query rows per KV group are processed together.  Scaled queries must lie in
 * the fp16 range (always true for fp16 queries).  Same reference semantics as
 * ss_decode_attn_dense (kernels.py:142-223, 303-378; attention.py:199-305).
 */
int ss_decode_attn_il8(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                       int n_kv_heads, int64_t t_q, int head_dim, float scale,
                       const int32_t *perm, const void *codebook, int n_blocks,
                       int n_centroids, const uint8_t *idx, const void *values_il8,
                       int v_dtype, int64_t cap, int64_t t_kv, int causal, int64_t q_offset,
                       void *out, int out_dtype, void *workspace, size_t workspace_bytes,
                       int n_splits, void *stream);

/*
 * ss_decode_attn_il8 over a hybrid cache whose compressed tokens keep fp16
 * values (value_backend "fp16"): compressed tokens 0 .. t_kv-1 plus the
 * recent-token buffer of t_buf tokens at positions t_kv .. t_kv+t_buf-1, in
 * one online softmax, with the buffer conventions of
 * ss_decode_attn_grouped_il_hybrid (keys and values in the original basis,
 * buf_dtype elements at k_buf/v_buf[b*buf_sb + h*buf_sh + t*buf_st + d]).
 * No reference counterpart: the reference takes a buffered hybrid cache to
 * its two-pass path (attention.py:238, 307-350), whose result this equals
 * within the decode tolerance.  t_buf = 0 is ss_decode_attn_il8.
 *   k_heavy  NULL, or fp16 [batch][n_kv_heads][cap][n_heavy_dims] (16-byte
 *            aligned rows, n_heavy_dims a multiple of 8, at most 32): the
 *            heavy blocks' key dims of a mixed-precision codec (codec basis,
 *            dims heavy_dims[], device int32), scored exactly on the matrix
 *            cores beside the LUT; the codebook must then hold zeros for
 *            those blocks (as SunShapeBlockCodec.scoring_centroids does).
 *            The same arguments follow t_buf in ss_decode_attn_grouped_il_hybrid
 *            (not for 4-bit codes at head_dim 128: SS_ERR_UNSUPPORTED),
 *            ss_decode_attn_turboquant_il (at most 32 dims) and
 *            ss_decode_attn_turboquant (at most 64; there the float32
 *            centroids' heavy blocks are skipped by the kernel).
 */
int ss_decode_attn_il8_hybrid(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                              int n_kv_heads, int64_t t_q, int head_dim, float scale,
                              const int32_t *perm, const void *codebook, int n_blocks,
                              int n_centroids, const uint8_t *idx, const void *values_il8,
                              int v_dtype, int64_t cap, int64_t t_kv, const void *k_buf,
                              const void *v_buf, int buf_dtype, int64_t buf_sb, int64_t buf_sh,
                              int64_t buf_st, int64_t t_buf, const void *k_heavy,
                              const int32_t *heavy_dims, int n_heavy_dims, int causal,
                              int64_t q_offset, void *out, int out_dtype, void *workspace,
                              size_t workspace_bytes, int n_splits, void *stream);

/*
 * Causal (or unmasked) attention of a prompt's T_q query rows per head
 * against an ss_decode_attn_il8 cache (same arguments and layouts, no
 * workspace): the shape of the reference's fused causal kernels at T_q > 1
 * (kernels.py:303-378; attention.py:244-298 with mask "causal").  Keys are
 * reconstructed from the prepared split-fp16 codebook (held in LDS) and
 * Q.K^T and P.V both run on the matrix cores; every workgroup takes
 * ss_prefill_rows_per_workgroup() query rows of one KV group (its rep query
 * heads at consecutive positions; twice that many for fp16 and bf16
 * queries, whose waves take 32 rows; bf16 queries are taken as fp16, exact
 * within fp16's range and saturating beyond +-65504), so the GQA group size
 * must divide that number.
 * head_dim 128, 16 blocks of 8, <= 256 centroids, fp16 values.
 * Row i of a head (position q_offset + i) sees keys 0 .. q_offset + i when
 * causal.  Results equal ss_decode_attn_il8's within the decode tolerance.
 */
int ss_prefill_rows_per_workgroup(void);
int ss_prefill_attn_il8(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                        int n_kv_heads, int64_t t_q, int head_dim, float scale,
                        const int32_t *perm, const void *codebook, int n_blocks,
                        int n_centroids, const uint8_t *idx, const void *values_il8,
                        int v_dtype, int64_t cap, int64_t t_kv, int causal, int64_t q_offset,
                        void *out, int out_dtype, void *stream);

/*
 * ss_prefill_attn_il8 over a hybrid cache: keys at positions 0 .. t_raw0 - 1
 * are indices (idx, capacity cap), keys at t_raw0 .. t_kv - 1 (its buffered
 * full-precision tokens) are given whole in kraw [batch][n_kv_heads]
 * [t_kv - t_raw0][2][128] fp16: per token its key in the codec's basis (the
 * permutation applied, or the rotation), times 2^-s, as fp16 (row 0) and
 * the fp16 remainder (row 1), with kfac[...][token] = 2^s (float32), s
 * chosen per token (ss_raw_key_rows) so the rows hold the key exactly (fp16
 * or bf16 keys) or to 22 bits (float32 keys).  values_il8 [batch][n_kv_heads][cap_v/8]
 * [128][8] holds the values of all t_kv tokens.  Replaces the reference's
 * two-pass path for prompts against a cache with buffered tokens
 * (attention.py:307-350, keys scored against the unpermuted query at
 * attention.py:318-321; the result is the same as scoring the whole key in
 * the codec's basis).  fp16 and bf16 queries only.
 */
int ss_prefill_attn_il8_hybrid(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                               int n_kv_heads, int64_t t_q, int head_dim, float scale,
                               const int32_t *perm, const void *codebook, int n_blocks,
                               int n_centroids, const uint8_t *idx, int64_t cap,
                               const void *values_il8, int64_t cap_v, int64_t t_kv,
                               const void *kraw, const float *kfac, int64_t t_raw0, int causal,
                               int64_t q_offset, void *out, int out_dtype, void *stream);

/*
 * ss_decode_attn_il8 without a workspace: the same kernel, arguments and
 * result, with its split partials and per-column split counters in a static
 * device array of the library (ss_decode_static_scratch_bytes() = 4 MiB,
 * one per GPU, held until the process ends).  The call allocates nothing
 * (no hipMalloc, no allocating library routine), for callers that cannot
 * allocate: code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation.  No counterpart in the reference.
 *  - A shape whose split scratch exceeds the static array returns
 *    SS_ERR_WORKSPACE (pass fewer splits, or use ss_decode_attn_il8).
 *  - The first call on a device looks the array up and clears its counter
 *    area with a fill kernel on `stream`, and the first call of a kernel
 *    variant sets its dynamic-LDS attribute; every completed call leaves the
 *    counters zero again.  Under HIP graph capture that set-up would only
 *    run at replay (and the attribute call may be refused), so make one
 *    eager call with the shape's query dtype before capturing; captured
 *    calls then record the decode kernel alone and replay unchanged.
 *  - All calls on one GPU share the array: calls that overlap in time on
 *    the same GPU (different streams or threads) race and give undefined
 *    results.
 */
int ss_decode_attn_il8_noalloc(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                               int n_kv_heads, int64_t t_q, int head_dim, float scale,
                               const int32_t *perm, const void *codebook, int n_blocks,
                               int n_centroids, const uint8_t *idx, const void *values_il8,
                               int v_dtype, int64_t cap, int64_t t_kv, int causal,
                               int64_t q_offset, void *out, int out_dtype, int n_splits,
                               void *stream);

/* Bytes of the static scratch array of ss_decode_attn_il8_noalloc (4 MiB). */
size_t ss_decode_static_scratch_bytes(void);

/*
 * KV append of values into the 8-token interleaved fp16 layout read by
 * ss_decode_attn_il8: token (b,h,t) of values (element j at
 * values[b*v_sb + h*v_sh + t*v_st + j]) is written at cache position
 * offset + t of out_il8 [n_b][n_h][cap/8][head_dim][8].  Replaces the value
 * half of update_and_fetch (reference cache.py:196-200).
 */
int ss_append_values_il8(const void *values, int v_dtype, int64_t n_b, int64_t n_h,
                         int64_t n_t, int64_t v_sb, int64_t v_sh, int64_t v_st,
                         int head_dim, void *out_il8, int64_t cap, int64_t offset,
                         void *stream);

/*
 * The whole KV append of an fp16-value cache (reference
 * SunShapeKVCache.update_and_fetch, cache.py:156-205, which quantises per
 * (batch, head) on the host and re-uploads every buffer): n_b x n_h x n_t
 * tokens of keys (strides k_*) are encoded as ss_encode_blockvq does into
 * rows offset .. offset + n_t of idx_cache [n_b][n_h][cap][n_blocks], and
 * their values (strides v_*) are stored as ss_append_values_il8 does into
 * values_il8 [n_b][n_h][cap/8][head_dim][8].  A decode step's few tokens take
 * one launch (a wave per (token, block) beside the value stores); a prompt
 * (more than 4096 token-blocks) takes the bulk encoders (the matrix-core one
 * with `prepared`, ss_encode_codebook's buffer, may be NULL) and then the
 * value stores.  Indices are identical to ss_encode_blockvq's.
 */
int ss_append_kv_il8(const void *keys, int keys_dtype, const void *values, int v_dtype,
                     int64_t n_b, int64_t n_h, int64_t n_t, int64_t k_sb, int64_t k_sh,
                     int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st, int head_dim,
                     const int32_t *perm, const float *centroids, int n_blocks,
                     int n_centroids, int block_dim, const void *prepared,
                     uint8_t *idx_cache, void *values_il8, int64_t cap, int64_t offset,
                     void *stream);

/*
 * One decode step of a hybrid cache with grouped 2/4-bit values kept in the
 * interleaved code layout (ss_pack_grouped_il), in one launch (reference
 * HybridSunShapeKVCache.update_and_fetch + _flush_buffer, cache.py:463-710,
 * which shifts the buffer and re-quantises per (batch, head) on the host):
 *   - n_new new tokens (keys/values strides k_*, v_*, dtype kv_dtype) are
 *     stored at buffer positions put_pos .. of buf_keys / buf_values
 *     [n_b][n_h][buf_cap][head_dim] (dtype buf_dtype);
 *   - the n_flush buffered tokens at positions flush_pos .. are encoded as
 *     ss_encode_blockvq does into rows offset .. of idx_cache
 *     [n_b][n_h][cap][n_blocks], and their values quantised as
 *     ss_quantize_values_grouped does (identical codes, scale and zero) into
 *     codes_il [n_b][n_h][cap / (32 / bits)][head_dim] (bits of other tokens
 *     kept) and scales / zeros [n_b][n_h][cap][head_dim / group_size].
 * The stored and flushed buffer ranges must not overlap.  Codecs with
 * block_dim 8 and at most 256 centroids; a step of more than 65536 flushed
 * token-blocks returns SS_ERR_UNSUPPORTED (take the separate appends).
 */
int ss_hybrid_append_grouped_il(
    const void *keys, const void *values, int kv_dtype, int64_t n_b, int64_t n_h, int64_t n_new,
    int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st,
    void *buf_keys, void *buf_values, int buf_dtype, int64_t buf_cap, int64_t put_pos,
    int64_t flush_pos, int64_t n_flush, int head_dim, const int32_t *perm, const float *centroids,
    int n_blocks, int n_centroids, int block_dim, uint8_t *idx_cache, int bits, int group_size,
    uint32_t *codes_il, void *scales, void *zeros, int sz_dtype, int64_t cap, int64_t offset,
    void *stream);

/*
 * As ss_decode_attn_dense with grouped asymmetric-quantised values decoded in
 * registers: v = ((w >> ((d % vpw) * bits)) & (2^bits - 1)) * scale + zero.
 * Replaces fused_attention_dequant_metal / _causal_metal (reference
 * kernels.py:697-765, 870-928).
 *   packed  uint32 [batch][n_kv_heads][cap][packed_dim], vpw = 32 / bits
 *           (2-bit: 16, 3-bit: 10, 4-bit: 8 values per word)
 *   scales, zeros  [batch][n_kv_heads][cap][head_dim / group_size], sz_dtype
 *                  (SS_F32 as the reference stores them, or SS_F16)
 */
int ss_decode_attn_grouped(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                           int n_kv_heads, int64_t t_q, int head_dim, float scale,
                           const int32_t *perm, const float *centroids, int n_blocks,
                           int n_centroids, const uint8_t *idx, const uint32_t *packed,
                           const void *scales, const void *zeros, int sz_dtype,
                           int bits, int group_size, int64_t cap, int64_t t_kv,
                           int causal, int64_t q_offset, void *out, int out_dtype,
                           void *workspace, size_t workspace_bytes, int n_splits,
                           void *stream);

/*
 * ss_decode_attn_grouped and ss_decode_attn_dense over a hybrid cache: the
 * recent-token buffer (k_buf / v_buf, buf_dtype SS_F16 / SS_BF16 / SS_F32,
 * element j of token t of (b, h) at b*buf_sb + h*buf_sh + t*buf_st + j,
 * original basis) joins the same softmax as positions t_kv .. t_kv + t_buf - 1
 * (one more split partial: fp32 dot products with the unpermuted scaled
 * query, online softmax over 256-token chunks).  The reference runs its
 * two-pass path whenever the buffer holds tokens (attention.py:238,
 * 307-350).  Workspace: ss_decode_turboquant_workspace_bytes(..., t_buf, ...)
 * bytes, the same layout.
 */
int ss_decode_attn_grouped_hybrid(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const float *centroids, int n_blocks,
    int n_centroids, const uint8_t *idx, const uint32_t *packed, const void *scales,
    const void *zeros, int sz_dtype, int bits, int group_size, int64_t cap, int64_t t_kv,
    const void *k_buf, const void *v_buf, int buf_dtype, int64_t buf_sb, int64_t buf_sh,
    int64_t buf_st, int64_t t_buf, int causal, int64_t q_offset, void *out, int out_dtype,
    void *workspace, size_t workspace_bytes, int n_splits, void *stream);
int ss_decode_attn_dense_hybrid(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const float *centroids, int n_blocks,
    int n_centroids, const uint8_t *idx, const void *values, int v_dtype, int64_t cap,
    int64_t t_kv, const void *k_buf, const void *v_buf, int buf_dtype, int64_t buf_sb,
    int64_t buf_sh, int64_t buf_st, int64_t t_buf, int causal, int64_t q_offset, void *out,
    int out_dtype, void *workspace, size_t workspace_bytes, int n_splits, void *stream);

/*
 * As ss_decode_attn_dense with TurboQuant values (reference
 * value_codecs.py:136-177): token t's value is norms[t] * (levels[code_t] @
 * rotation), code_t its packed BITS-bit codes.  The reference has no fused
 * kernel for these values: it dequantises the whole cache every step and
 * runs the two-pass SDPA (cache.py:774-784, attention.py:307-350), which this
 * replaces.  Accumulation runs in the rotated basis; the rotation is applied
 * once per output row (a later launch on the same stream).  A hybrid cache's
 * t_buf buffered tokens (k_buf/v_buf, original basis, element j of token t of
 * (b, h) at [b*buf_sb + h*buf_sh + t*buf_st + j], buf_dtype f16/bf16/f32)
 * join the same softmax as positions t_kv .. t_kv + t_buf - 1, as one more
 * split partial taken into the rotated basis (reference attention.py:238
 * sends such caches to the two-pass path instead).
 *   packed    uint32 [batch][n_kv_heads][cap][packed_dim], pack_indices layout
 *   norms     float  [batch][n_kv_heads][cap]
 *   levels    HOST float[2^bits], ascending Lloyd-Max levels x 1/sqrt(head_dim)
 *   rotation  float  [head_dim][head_dim] (device), unit = rotated @ rotation
 *   workspace ss_decode_turboquant_workspace_bytes(...) bytes, 256-byte
 *             aligned, always required (it holds the rotated-basis rows)
 */
int ss_decode_attn_turboquant(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                              int n_kv_heads, int64_t t_q, int head_dim, float scale,
                              const int32_t *perm, const float *centroids, int n_blocks,
                              int n_centroids, const uint8_t *idx, const uint32_t *packed,
                              const float *norms, const float *levels, const float *rotation,
                              int bits, int64_t cap, int64_t t_kv, const void *k_buf,
                              const void *v_buf, int buf_dtype, int64_t buf_sb,
                              int64_t buf_sh, int64_t buf_st, int64_t t_buf,
                              const void *k_heavy, const int32_t *heavy_dims, int n_heavy_dims,
                              int causal, int64_t q_offset, void *out, int out_dtype,
                              void *workspace, size_t workspace_bytes, int n_splits,
                              void *stream);
size_t ss_decode_turboquant_workspace_bytes(int64_t batch, int n_q_heads, int n_kv_heads,
                                            int64_t t_q, int head_dim, int64_t t_kv,
                                            int64_t t_buf, int n_splits);

/*
 * ss_decode_attn_turboquant for 2-bit codes held token-interleaved, on the
 * matrix cores (the same replacement of the reference's TurboQuant two-pass
 * path, value_codecs.py:136-177 with attention.py:307-350): the LUT is built
 * from the prepared codebook (ss_codebook_f16x2) and P.V runs as
 * v_mfma_f32_16x16x32_bf16 products, using that a symmetric 2-bit level
 * table is affine in the two code bits (levels[3] = levels[2] + levels[1] -
 * levels[0], else SS_ERR_UNSUPPORTED).  Arguments as ss_decode_attn_turboquant
 * except:
 *   codebook  ss_codebook_f16x2 of the key centroids (16-byte aligned)
 *   codes_il  uint32 [batch][n_kv_heads][cap/16][head_dim], the layout of
 *             ss_decode_attn_grouped_il's 2-bit words (ss_pack_grouped_il
 *             writes it from pack_indices rows); cap % 16 == 0
 *   norms     float [batch][n_kv_heads][cap], 16-byte aligned
 *   levels    HOST float[4]
 */
int ss_decode_attn_turboquant_il(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                                 int n_kv_heads, int64_t t_q, int head_dim, float scale,
                                 const int32_t *perm, const void *codebook, int n_blocks,
                                 int n_centroids, const uint8_t *idx, const uint32_t *codes_il,
                                 const float *norms, const float *levels, const float *rotation,
                                 int64_t cap, int64_t t_kv, const void *k_buf, const void *v_buf,
                                 int buf_dtype, int64_t buf_sb, int64_t buf_sh, int64_t buf_st,
                                 int64_t t_buf, const void *k_heavy, const int32_t *heavy_dims,
                                 int n_heavy_dims, int causal, int64_t q_offset, void *out,
                                 int out_dtype, void *workspace, size_t workspace_bytes,
                                 int n_splits, void *stream);

/*
 * As ss_decode_attn_turboquant with SunShape block-VQ values (value backend
 * "sunshape", reference cache.py:614-623): token t's value is the value
 * codec's dequantisation of its indices, concat_b v_centroids[b][v_idx[t][b]]
 * taken back to the original basis by v_transform.  The reference has no
 * fused kernel for these values: it dequantises the whole cache on the CPU
 * every step (cache.py:785-800) and runs the two-pass SDPA.
 *   v_idx        uint8 [batch][n_kv_heads][cap][head_dim / v_block_dim]
 *   v_centroids  float [head_dim / v_block_dim][v_n_centroids][v_block_dim],
 *                v_block_dim 4 or 8, v_n_centroids <= 256
 *   v_transform  float [head_dim][head_dim] (device): original = codec-space
 *                row @ v_transform (the inverse permutation as a 0/1 matrix,
 *                or the codec rotation)
 *   k_heavy      NULL, or fp16 [batch][n_kv_heads][cap][n_heavy_dims]: the
 *                heavy blocks' key dims of a mixed-precision codec (codec
 *                basis), scored exactly in place of the LUT; heavy_dims
 *                int32 [n_heavy_dims] are their codec-basis dims
 *                (n_heavy_dims a multiple of 8, at most 64).  Every block
 *                holding a heavy dim leaves the centroid sum, whatever its
 *                centroids hold.  The reference zeroes these blocks'
 *                centroids at fit time (codec.py:381-388; its DSQ
 *                refinement can move them again, codec.py:400-410) and
 *                scores index 0 of them, although its README calls them
 *                fp16 blocks; NULL keeps the reference's scores.
 *   workspace    ss_decode_turboquant_workspace_bytes(...) bytes (same layout)
 */
int ss_decode_attn_sunshape_v(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                              int n_kv_heads, int64_t t_q, int head_dim, float scale,
                              const int32_t *perm, const float *centroids, int n_blocks,
                              int n_centroids, const uint8_t *idx, const uint8_t *v_idx,
                              const float *v_centroids, int v_block_dim, int v_n_centroids,
                              const float *v_transform, const void *k_heavy,
                              const int32_t *heavy_dims, int n_heavy_dims, int64_t cap,
                              int64_t t_kv,
                              const void *k_buf, const void *v_buf, int buf_dtype,
                              int64_t buf_sb, int64_t buf_sh, int64_t buf_st, int64_t t_buf,
                              int causal, int64_t q_offset, void *out, int out_dtype,
                              void *workspace, size_t workspace_bytes, int n_splits,
                              void *stream);

/*
 * As ss_decode_attn_grouped with the 2- or 4-bit codes held in a token-
 * interleaved layout and the codebook prepared by ss_codebook_f16x2.  Code of
 * token t, dimension d of a (batch, KV head) row is the bits-wide field at
 * bit bits*(i/2) + 16*(i%2), i = t%tpw, of
 * codes_il[((b*n_kv_heads + h)*cap/tpw + t/tpw)*head_dim + d], tpw = 32/bits
 * (even tokens of the word in its low half, odd tokens in its high half);
 * scales/zeros keep ss_decode_attn_grouped's [batch][n_kv_heads][cap][n_groups]
 * layout.  group_size must be head_dim or head_dim/2, cap % 16 == 0, all
 * operands 16-byte aligned.  The LUT and P.V run on the matrix cores (P.V in
 * bf16 on the codes with p*scale split into bf16 hi/lo parts, the zero term
 * added exactly in fp32).  Replaces fused_attention_dequant_metal /
 * _causal_metal (reference kernels.py:697-765, 870-928).
 */
int ss_decode_attn_grouped_il(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                              int n_kv_heads, int64_t t_q, int head_dim, float scale,
                              const int32_t *perm, const void *codebook, int n_blocks,
                              int n_centroids, const uint8_t *idx, const uint32_t *codes_il,
                              const void *scales, const void *zeros, int sz_dtype, int bits,
                              int group_size, int64_t cap, int64_t t_kv, int causal,
                              int64_t q_offset, void *out, int out_dtype, void *workspace,
                              size_t workspace_bytes, int n_splits, void *stream);

/*
 * ss_decode_attn_grouped_il over a hybrid cache: the compressed tokens
 * 0 .. t_kv-1 plus the cache's recent-token buffer of t_buf tokens at
 * positions t_kv .. t_kv+t_buf-1, in one online softmax.  Buffer keys and
 * values are in the original (unpermuted, unrotated) basis, buf_dtype
 * (SS_F16/SS_BF16/SS_F32) elements at k_buf/v_buf[b*buf_sb + h*buf_sh +
 * t*buf_st + d] (strides in elements, multiples of 8; k_buf 16-byte
 * aligned); their scores are fp32 dot products with round_to(q_dtype,
 * q*scale).  No reference counterpart: the reference's fused path takes
 * only an empty buffer and otherwise falls back to the two-pass path
 * (attention.py:238); the result equals that two-pass path's
 * (attention.py:307-350) within the decode tolerance.
 */
int ss_decode_attn_grouped_il_hybrid(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                                     int n_kv_heads, int64_t t_q, int head_dim, float scale,
                                     const int32_t *perm, const void *codebook, int n_blocks,
                                     int n_centroids, const uint8_t *idx,
                                     const uint32_t *codes_il, const void *scales,
                                     const void *zeros, int sz_dtype, int bits, int group_size,
                                     int64_t cap, int64_t t_kv, const void *k_buf,
                                     const void *v_buf, int buf_dtype, int64_t buf_sb,
                                     int64_t buf_sh, int64_t buf_st, int64_t t_buf,
                                     const void *k_heavy, const int32_t *heavy_dims,
                                     int n_heavy_dims, int causal, int64_t q_offset, void *out,
                                     int out_dtype, void *workspace, size_t workspace_bytes,
                                     int n_splits, void *stream);

/*
 * Repack grouped codes (pack_indices words, one row of packed_dim words per
 * token: word w of token (b,h,t) at packed[b*p_sb + h*p_sh + t*p_st + w]) into
 * the interleaved layout of ss_decode_attn_grouped_il at cache positions
 * offset .. offset+n_t-1 of out_il [n_b][n_h][cap/tpw][head_dim]; other
 * tokens sharing a word keep their codes.  Replaces the value-code half of
 * the hybrid cache flush (reference cache.py:581-596).
 */
int ss_pack_grouped_il(const uint32_t *packed, int64_t n_b, int64_t n_h, int64_t n_t,
                       int64_t p_sb, int64_t p_sh, int64_t p_st, int head_dim, int bits,
                       uint32_t *out_il, int64_t cap, int64_t offset, void *stream);

/*
 * One decode step of an fp16-value cache in one launch: the cache holds
 * t_cache tokens (idx [batch][n_kv_heads][cap][n_blocks], values_il8 as
 * ss_decode_attn_il8), and the step's n_new (1..4) new tokens arrive as fp16
 * keys / values at k_new / v_new [b*kv_sb + h*kv_sh + j*kv_st + dim].  The
 * kernel encodes the new keys (indices identical to ss_append_kv_il8's:
 * key . centroid products on the matrix cores from the prepared codebook,
 * accepted under a proven float error bound, else ranked exactly over the
 * float32 centroids), attends all t_cache + n_new tokens as
 * ss_decode_attn_il8 would after the append (the new tokens' weights and
 * values in float32), and stores the new tokens' index rows and values at
 * positions t_cache .. t_cache + n_new - 1.  Replaces the reference's decode
 * step, update_and_fetch (cache.py:156-205) followed by the fused attention
 * (kernels.py:142-230, attention.py:236-305), which touch the cache twice.
 * Other arguments as ss_decode_attn_il8; centroids float32
 * [n_blocks][n_centroids][8] (16-byte aligned), codebook their
 * ss_codebook_f16x2.  Calls sharing a cache must not overlap.
 */
int ss_decode_step_il8(const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads,
                       int64_t t_q, int head_dim, float scale, const int32_t *perm,
                       const void *codebook, const float *centroids, int n_blocks,
                       int n_centroids, uint8_t *idx, void *values_il8, int64_t cap,
                       int64_t t_cache, const void *k_new, const void *v_new, int kv_dtype,
                       int64_t kv_sb, int64_t kv_sh, int64_t kv_st, int64_t n_new, int causal,
                       int64_t q_offset, void *out, int out_dtype, void *workspace,
                       size_t workspace_bytes, int n_splits, void *stream);

/*
 * One decode step of a hybrid cache with 2- or 4-bit interleaved grouped
 * values (ss_decode_attn_grouped_il_hybrid's layouts) in one launch.  The cache holds
 * t_kv (>= 1) compressed tokens and n_buf buffered float16 tokens, the buffer
 * window at k_buf / v_buf [b*buf_sb + h*buf_sh + row*buf_st + dim], rows 0 ..
 * n_buf-1 oldest first; the step's n_new (1..4) float16 tokens arrive at
 * k_new / v_new [b*kv_sb + h*kv_sh + j*kv_st + dim].  As the reference's
 * HybridSunShapeKVCache.update_and_fetch (cache.py:656-710) followed by its
 * attention (attention.py:307-350), the n_flush (0..4, <= n_buf) oldest
 * buffered tokens move into compressed storage and the new tokens into the
 * buffer, and every token is attended: the kernel encodes the flushed keys
 * (indices identical to ss_hybrid_append_grouped_il's, as ss_decode_step_il8
 * encodes), quantises their values with the grouped min/max rule (codes,
 * scale and zero identical to it), attends them in that compressed form at
 * positions t_kv .., the remaining buffered and the new tokens exactly after
 * them, and stores the flushed tokens' index rows, codes, scales and zeros
 * at positions t_kv .. t_kv + n_flush - 1 and the new tokens at buffer rows
 * n_buf .. n_buf + n_new - 1 (the caller's buffer store must hold them).
 * Other arguments as ss_decode_attn_grouped_il; centroids float32
 * [n_blocks][n_centroids][8] (16-byte aligned), codebook their
 * ss_codebook_f16x2.  The caller then counts t_kv + n_flush compressed and
 * n_buf - n_flush + n_new buffered tokens, the window starting n_flush rows
 * later.  Calls sharing a cache must not overlap.
 */
int ss_decode_step_grouped_il_hybrid(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const void *codebook, const float *centroids,
    int n_blocks, int n_centroids, uint8_t *idx, uint32_t *codes_il, void *scales, void *zeros,
    int sz_dtype, int bits, int group_size, int64_t cap, int64_t t_kv, void *k_buf, void *v_buf,
    int buf_dtype, int64_t buf_sb, int64_t buf_sh, int64_t buf_st, int64_t n_buf, int64_t n_flush,
    const void *k_new, const void *v_new, int kv_dtype, int64_t kv_sb, int64_t kv_sh, int64_t kv_st,
    int64_t n_new, int causal, int64_t q_offset, void *out, int out_dtype, void *workspace,
    size_t workspace_bytes, int n_splits, void *stream);

/*
 * The same step for a hybrid cache with fp16 values held 8-token interleaved
 * (ss_decode_attn_il8_hybrid's layouts, value_backend "fp16"): the flushed
 * tokens' keys are encoded as above, their fp16 values attended as they are
 * and stored into values_il8 at positions t_kv .. (as ss_append_values_il8);
 * the rest as ss_decode_step_grouped_il_hybrid.  Replaces the reference's
 * HybridSunShapeKVCache.update_and_fetch (cache.py:656-710) and its two-pass
 * attention (attention.py:307-350) for such caches.
 */
int ss_decode_step_il8_hybrid(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const void *codebook, const float *centroids,
    int n_blocks, int n_centroids, uint8_t *idx, void *values_il8, int64_t cap, int64_t t_kv,
    void *k_buf, void *v_buf, int buf_dtype, int64_t buf_sb, int64_t buf_sh, int64_t buf_st,
    int64_t n_buf, int64_t n_flush, const void *k_new, const void *v_new, int kv_dtype,
    int64_t kv_sb, int64_t kv_sh, int64_t kv_st, int64_t n_new, int causal, int64_t q_offset,
    void *out, int out_dtype, void *workspace, size_t workspace_bytes, int n_splits, void *stream);

/*
 * The inverse of ss_pack_grouped_il: the first n_t tokens of interleaved
 * codes codes_il [n_bh][cap/tpw][head_dim] (n_bh = batch x heads rows) as
 * pack_indices rows out [n_bh][n_t][head_dim*bits/32].  Replaces the
 * reference's values_packed_raw accessor (cache.py:858-866), whose rows
 * this layout stores rearranged; bits 2 or 4.
 */
int ss_grouped_il_to_packed(const uint32_t *codes_il, int64_t n_bh, int64_t cap, int head_dim,
                            int bits, int64_t n_t, uint32_t *out, void *stream);

/*
 * Dequantise the first n_t tokens of interleaved grouped codes (codes_il as
 * above; scales/zeros [n_bh][sz_cap][head_dim/group_size], f32 or f16)
 * straight into the 8-token interleaved fp16 layout out_il8
 * [n_bh][cap_out/8][head_dim][8] at positions 0 .. n_t-1, for the hybrid
 * prompt kernel (ss_prefill_attn_il8_hybrid).  v = fp16(q*scale + zero), the
 * product and the sum rounded in float32 as dequantize_values (reference
 * kernels.py:1231-1269) does before the cast.  Positions n_t .. of the last
 * 8-token group are written as zero; later groups are not written.
 */
int ss_grouped_il_to_il8(const uint32_t *codes_il, int64_t n_bh, int64_t cap, int head_dim,
                         int bits, int group_size, const void *scales, const void *zeros,
                         int sz_dtype, int64_t sz_cap, int64_t n_t, void *out_il8,
                         int64_t cap_out, void *stream);

/*
 * The whole-key rows kraw / kfac of ss_prefill_attn_il8_hybrid from buffered
 * keys: token (b,h,t) reads keys[b*k_sb + h*k_sh + t*k_st + perm[j]] for dim
 * j (perm NULL = identity), writes rows [n_b][n_h][n_t][2][head_dim] fp16
 * and factors [n_b][n_h][n_t] float32 as described there, s from max |key|.
 * No counterpart in the reference (its two-pass path, attention.py:307-350,
 * multiplies the buffered fp16 keys directly); one launch per prompt.
 */
int ss_raw_key_rows(const void *keys, int k_dtype, int64_t n_b, int64_t n_h, int64_t n_t,
                    int64_t k_sb, int64_t k_sh, int64_t k_st, int head_dim, const int32_t *perm,
                    void *rows, float *factors, void *stream);

/*
 * Grouped asymmetric min-max quantisation of values (encode-on-append).
 * Replaces quantize_values (reference kernels.py:1173-1228): per token and
 * group, zero = min, scale = max((max - min) / (2^bits - 1), 1e-8),
 * q = clip(rint((v - zero) / scale), 0, 2^bits - 1), packed as pack_indices.
 * Token (b,h,t) reads values[b*v_sb + h*v_sh + t*v_st + j] (elements) and
 * writes packed[(b*o_sb + h*o_sh + t*o_st)*packed_dim + w] and
 * scales/zeros[(b*o_sb + h*o_sh + t*o_st)*n_groups + g] (token-row strides
 * o_* counted in tokens).  Codes use the float32 scale/zero; they are stored
 * in sz_dtype.
 */
int ss_quantize_values_grouped(const void *values, int v_dtype, int64_t n_b,
                               int64_t n_h, int64_t n_t, int64_t v_sb, int64_t v_sh,
                               int64_t v_st, int head_dim, int bits, int group_size,
                               uint32_t *packed, void *scales, void *zeros,
                               int sz_dtype, int64_t o_sb, int64_t o_sh,
                               int64_t o_st, void *stream);

/* v[t][d] = q * scale + zero (separate float32 multiply and add), out_dtype.
 * Replaces dequantize_values (reference kernels.py:1231-1269).  Rows are
 * contiguous: packed [n_tok][packed_dim], scales/zeros [n_tok][n_groups],
 * out [n_tok][head_dim]. */
int ss_dequantize_values_grouped(const uint32_t *packed, const void *scales,
                                 const void *zeros, int sz_dtype, int64_t n_tok,
                                 int head_dim, int bits, int group_size, void *out,
                                 int out_dtype, void *stream);

/* Bit packing of small codes into uint32 words (reference kernels.py:1102-1163).
 * in: uint8 [n_rows][d]; out: uint32 [n_rows][packed_dim(d, bits)]. */
int ss_pack_indices(const uint8_t *in, int64_t n_rows, int d, int bits, uint32_t *out,
                    void *stream);
/* out: uint32 [n_rows][d]. */
int ss_unpack_indices(const uint32_t *in, int64_t n_rows, int d, int bits,
                      uint32_t *out, void *stream);

/* idx[i] = #{b : v[i] > boundaries[b]} as uint8 (reference kernels.py:453-507).
 * values float32 [n]; boundaries float32 [n_boundaries] (device). */
int ss_scalar_quantize(const float *values, int64_t n, const float *boundaries,
                       int n_boundaries, uint8_t *out, void *stream);

/* Block-VQ decode k_hat[t][inv_perm...]: out[t][j] = C[b][idx[t][b]][d] placed at
 * codec position j = b*bd + d, then out_orig[t][i] = out[t][inv_perm[i]]
 * (inv_perm may be NULL).  Replaces codec.dequantize (reference
 * codec.py:516-543) and the key reconstruction of cache.py:211-240.
 * idx uint8 row stride in bytes; out [n_tok][head_dim] out_dtype. */
int ss_dequantize_blockvq(const uint8_t *idx, int64_t n_tok, int64_t idx_row_stride,
                          const float *centroids, int n_blocks, int n_centroids,
                          int block_dim, const int32_t *inv_perm, void *out,
                          int out_dtype, void *stream);

/*
 * Lloyd k-means of every codec block at once (codec fitting on the GPU;
 * replaces the per-block NumPy k-means of the reference's fit,
 * codec.py:53-103 called from codec.py:389-392).  One workgroup per block.
 *   data       float [n_blocks][n_points][block_dim] (block-major, contiguous)
 *   centroids  float [n_blocks][n_centroids][block_dim]: the initial
 *              centroids in (the reference draws them as data rows
 *              RandomState(seed + b).permutation(n)[:K]), the fitted ones out
 *   assign     uint8 [n_blocks][n_points] final assignments, or NULL
 * Each iteration: expanded-form float32 distances with first-index argmin,
 * per-centroid float32 sums in point order divided in double; empty clusters
 * keep their centroid.  block_dim 4 or 8, n_centroids <= 256 < n_points <=
 * 131072 (a block with no more points than centroids is the caller's
 * zero-padded codebook, as in the reference).
 */
int ss_kmeans_blocks(const float *data, int n_blocks, int64_t n_points, int block_dim,
                     int n_centroids, int iters, float *centroids, uint8_t *assign,
                     void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SUNSHAPE_HIP_H */
