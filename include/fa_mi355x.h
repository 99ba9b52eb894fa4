/*
 * fa_mi355x.h — C ABI of the MI355X (gfx950) attention path.
 *
 * This is the drop-in boundary that replaces the reference's torch extension
 * `flashattention_custom._ext` (csrc/ext.cpp:91-116). Every entry point takes
 * plain device pointers, sizes and an explicit HIP stream; nothing here
 * allocates or frees device memory, and no torch type crosses the boundary.
 *
 * Conventions
 *   - All tensors are dense, row-major ("contiguous") device buffers.
 *   - fp16 buffers hold IEEE binary16 values; int32 buffers hold int32_t.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream). Work is
 *     enqueued asynchronously; no entry point synchronises the host.
 *   - The current HIP device must be the device that owns the buffers.
 *   - Return value: 0 on success, a negative FA_ERR_* code otherwise; the
 *     message of the last failure on the calling thread is fa_last_error().
 *
 * Paged K/V layout (reference: csrc/flash_attn_sm75.cu:54-86, ops.py:34-45)
 *   k_pages, v_pages : fp16 [NB, Hk, P, PS, D]
 *   Token `pos` of sequence b lives in logical page pos / PS, slot pos % PS.
 *   Logical page p of sequence b maps to a physical page id phi:
 *     block_table == NULL : phi = b * P + p               (reference identity map)
 *     block_table != NULL : phi = block_table[b * max_blocks + p]
 *   and phi addresses k_pages[phi / P, hk, phi % P, :, :]. Physical ids outside
 *   [0, NB * P) and logical pages beyond the capacity (P, or max_blocks with a
 *   block table) are never dereferenced: they read as absent keys and are
 *   skipped on append.
 */
#ifndef FA_MI355X_H
#define FA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 4

/* element type of q / k / v / o */
#define FA_DTYPE_F16 0
#define FA_DTYPE_F32 1

/* status codes */
#define FA_OK 0
#define FA_ERR_INVALID -1   /* an argument failed validation            */
#define FA_ERR_LAUNCH  -2   /* the HIP runtime rejected a kernel launch */
#define FA_ERR_WORKSPACE -3 /* workspace missing or smaller than needed */

/*
 * Contiguous attention: O = softmax(Q K^T / sqrt(D) + causal mask) V.
 * Replaces _ext.flash_attn_fwd (csrc/ext.cpp:30-40) and its launcher
 * flash_attn_fwd_cuda (csrc/flash_attn_sm75.cu:428-467).
 *
 *   q, o : [B, Hq, M, D]     k, v : [B, Hk, N, D]     dtype: FA_DTYPE_F16 | FA_DTYPE_F32
 *   Hq % Hk == 0; q head h reads K/V head h / (Hq / Hk) (Hq == Hk is the
 *   reference's MHA case). D in {64, 128}.
 *   Key j is visible to query row i iff j < N and, when causal != 0,
 *   k_off + j <= q_off + i, where q_off = q_offsets ? q_offsets[b] : q_offset
 *   (likewise k_off). q_offsets / k_offsets are nullable int32 [B] buffers.
 *   A row with no visible key (N > 0) yields NaN, and N == 0 yields zeros, as
 *   in the reference's CPU math (flashattention_custom/ops.py:19-31).
 */
int fa_flash_attn_fwd(const void* q, const void* k, const void* v, void* o,
                      int dtype, int B, int Hq, int Hk, int M, int N, int D,
                      int causal, int64_t q_offset, int64_t k_offset,
                      const int32_t* q_offsets, const int32_t* k_offsets,
                      void* stream);

/*
 * fa_flash_attn_fwd with a workspace, so that calls with few query rows run
 * on the split-K decode kernels. The reference serves every M with one
 * launcher, grid (B, H, ceil(M/16)) (csrc/flash_attn_sm75.cu:428-467); here
 * fp16 calls with at most 32 query rows per K/V head (M * Hq/Hk <= 32, e.g.
 * single-token decode over a contiguous cache) split each K/V head's keys
 * over the whole device and merge the partial results in a second kernel,
 * while other calls take the prefill kernels exactly as fa_flash_attn_fwd
 * does. Arguments and results are fa_flash_attn_fwd's.
 *   workspace : device scratch of at least fa_flash_attn_workspace_bytes(...)
 *               bytes for the same sizes (may be NULL when that is 0); its
 *               contents need no initialisation.
 */
int fa_flash_attn_fwd_ws(const void* q, const void* k, const void* v, void* o,
                         int dtype, int B, int Hq, int Hk, int M, int N, int D,
                         int causal, int64_t q_offset, int64_t k_offset,
                         const int32_t* q_offsets, const int32_t* k_offsets,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * Workspace bytes fa_flash_attn_fwd_ws needs for these sizes (0: the call
 * runs on the prefill kernels and needs none). Host-known sizes only.
 */
size_t fa_flash_attn_workspace_bytes(int dtype, int B, int Hq, int Hk, int M, int N, int D);

/*
 * Paged attention over a K/V page pool (prefill chunk or single-token decode).
 * Replaces _ext.flash_attn_paged_fwd (csrc/ext.cpp:42-68) and its launcher
 * flash_attn_paged_fwd_cuda (csrc/flash_attn_sm75.cu:469-525).
 *
 *   q, o : fp16 [B, Hq, M, D]       k_pages, v_pages : fp16 [NB, Hk, P, PS, D]
 *   seqlen   : int32 [B]   number of cached tokens of sequence b (clamped to
 *                          the capacity P*PS, or max_blocks*PS)
 *   head_map : int32 [Hq]  K/V head read by each query head (reference
 *                          engine/llama_tp.py:145-156); an entry outside
 *                          [0, Hk) makes that head's output NaN.
 *   block_table : nullable int32 [B, max_blocks] (see header comment);
 *                 without it NB must equal B.
 *   Visibility and offsets as in fa_flash_attn_fwd with N = seqlen[b].
 *   q_lens   : nullable int32 [B]: only query rows i < q_lens[b] of sequence
 *              b are live (a ragged chunk padded to M rows); rows at or past
 *              it are not computed and come out as zeros. NULL: all M rows.
 *              An additive extension for chunked prefill with per-sequence
 *              offsets (the reference's generate loop, engine/llama_tp.py:
 *              338-354, runs equal-length chunks only).
 *   heads_per_kv : the most query heads head_map sends to one KV head
 *              (Hq/Hk for the usual GQA map hq // (Hq/Hk)); <= 0 means Hq,
 *              no assumption. It sizes the decode workspace, whose partial
 *              slots each hold one KV head's query rows, and, with M < 128
 *              off the decode path, lets the prefill kernel pack the
 *              (head, position) rows of a KV head's q heads into shared
 *              128-row tiles (one pass over the KV head's pages for all of
 *              them; <= 0 keeps one q head per tile). If head_map sends
 *              more heads to a KV head, the heads past the bound get NaN rows
 *              on both paths; nothing is written out of bounds.
 *   workspace : device scratch of at least fa_paged_workspace_bytes(...)
 *               bytes for the same arguments (may be NULL when that is 0);
 *               its contents need no initialisation.
 */
int fa_flash_attn_paged_fwd(const void* q, const void* k_pages, const void* v_pages,
                            const int32_t* seqlen, int page_size,
                            const int32_t* head_map, void* o,
                            int B, int Hq, int M, int D, int NB, int Hk, int P,
                            int causal, int64_t q_offset, int64_t k_offset,
                            const int32_t* q_offsets, const int32_t* k_offsets,
                            const int32_t* q_lens,
                            const int32_t* block_table, int max_blocks,
                            int heads_per_kv,
                            void* workspace, size_t workspace_bytes,
                            void* stream);

/*
 * fa_flash_attn_paged_fwd without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc). It has no counterpart in the reference, whose
 * launcher allocates its output with torch (csrc/flash_attn_sm75.cu:492).
 * It allocates nothing: the decode path's partial results go to a static
 * device array of 32 MiB per GPU, held until the process ends. Arguments and
 * results are those of fa_flash_attn_paged_fwd, except that shapes with more
 * than 64 query rows per KV head (M * ceil(Hq/Hk)) whose decode workspace
 * (fa_paged_workspace_bytes) exceeds 32 MiB run on the prefill kernel, which
 * needs none (same results within the fp32-softmax tolerance, not bit for
 * bit); other shapes beyond 32 MiB are rejected with FA_ERR_WORKSPACE before
 * anything is launched. All calls on one GPU share
 * its scratch, so calls that overlap on one GPU (concurrent streams, or
 * threads without ordering) race; calls ordered on one stream do not. The
 * scratch needs no initialisation and keeps the last call's contents.
 */
int fa_flash_attn_paged_fwd_noalloc(const void* q, const void* k_pages, const void* v_pages,
                                    const int32_t* seqlen, int page_size,
                                    const int32_t* head_map, void* o,
                                    int B, int Hq, int M, int D, int NB, int Hk, int P,
                                    int causal, int64_t q_offset, int64_t k_offset,
                                    const int32_t* q_offsets, const int32_t* k_offsets,
                                    const int32_t* q_lens,
                                    const int32_t* block_table, int max_blocks,
                                    int heads_per_kv, void* stream);

/*
 * Workspace bytes fa_flash_attn_paged_fwd needs for these shapes and this
 * heads_per_kv bound. It depends only on host-known sizes (the per-sequence
 * capacity in pages is P, or max_blocks when a block table is used), never on
 * device contents: (B*Hk + W) slots x heads_per_kv*M rows x (D + 2) fp32, W
 * the decode workgroup count (<= 1024), plus 2*B + 1 ints, with B capped at
 * 2048: a larger batch runs in decode launches of at most 2048 sequences one
 * after another, which share the workspace.
 */
size_t fa_paged_workspace_bytes(int B, int Hq, int M, int D, int Hk,
                                int capacity_pages, int page_size, int heads_per_kv);

/*
 * Write T new tokens per sequence into their pages, in place:
 *   k_pages[page(pos), hk, slot(pos), :] = k_new[b, hk, t, :]  (same for V),
 *   pos = start + t, start = start_positions ? start_positions[b] : start_pos.
 * Replaces _ext.paged_kv_append (csrc/ext.cpp:70-89) and paged_kv_append_cuda
 * with its kernel (csrc/flash_attn_sm75.cu:528-588).
 *   k_new, v_new : fp16 [B, Hk, T, D]    pages as above, D % 8 == 0.
 * Positions whose page is negative or beyond the capacity, or whose physical
 * page id is out of range, are skipped (reference kernel: :548).
 */
int fa_paged_kv_append(void* k_pages, void* v_pages,
                       const void* k_new, const void* v_new,
                       int B, int Hk, int T, int D, int NB, int P, int page_size,
                       int64_t start_pos, const int32_t* start_positions,
                       const int32_t* block_table, int max_blocks,
                       void* stream);

/*
 * fa_flash_attn_paged_fwd with the rotary embedding of Q applied at load
 * time: query row i of sequence b is rotated at position q_off(b) + i by the
 * half-split rule of engine/rope.py:15-24 (y1 = x1*c - x2*s, y2 = x1*s + x2*c
 * over the halves x1 = q[:D/2], x2 = q[D/2:], each product and sum rounded to
 * fp16 in the reference's order). Fuses the reference's apply_rope(q, ...)
 * (engine/llama_tp.py:182-183) into the attention prologue.
 *   rope_cos, rope_sin : fp16 [rope_len, D/2] (build_rope_cache, rope.py:6-13).
 * A row whose position is outside [0, rope_len) yields NaN.
 */
int fa_flash_attn_paged_rope_fwd(const void* q, const void* k_pages, const void* v_pages,
                                 const int32_t* seqlen, int page_size,
                                 const int32_t* head_map, void* o,
                                 int B, int Hq, int M, int D, int NB, int Hk, int P,
                                 int causal, int64_t q_offset, int64_t k_offset,
                                 const int32_t* q_offsets, const int32_t* k_offsets,
                                 const int32_t* q_lens,
                                 const int32_t* block_table, int max_blocks,
                                 int heads_per_kv,
                                 void* workspace, size_t workspace_bytes,
                                 const void* rope_cos, const void* rope_sin, int rope_len,
                                 void* stream);

/*
 * fa_paged_kv_append with the rotary embedding of K fused in: the key row of
 * token t is rotated at its position start + t (same rule and tables as
 * above; D % 16 == 0) before it is written; V is copied unchanged. Fuses
 * apply_rope(k, ...) and cache.append (engine/llama_tp.py:183-186) into one
 * pass. Keys at a position outside [0, rope_len) are written as NaN.
 */
int fa_paged_kv_append_rope(void* k_pages, void* v_pages,
                            const void* k_new, const void* v_new,
                            int B, int Hk, int T, int D, int NB, int P, int page_size,
                            int64_t start_pos, const int32_t* start_positions,
                            const int32_t* block_table, int max_blocks,
                            const void* rope_cos, const void* rope_sin, int rope_len,
                            void* stream);

/*
 * Write token t of sequence b at its own position positions[b * T + t], in
 * place (same K/V and page layouts as fa_paged_kv_append). Replaces the
 * general [B, T] path of the reference's cache, PagedKVCache.append
 * (engine/llama_tp.py:80-99), which scatters one (b, t) row at a time from
 * Python. One kernel launch; nothing is read back.
 *   positions : int32 [B, T] device buffer. A negative position, or one whose
 *               page is beyond the capacity or unmapped, is skipped. Two
 *               tokens of one sequence at the same position write the same
 *               slot in an unspecified order (the caller keeps the last one,
 *               as the reference's loop does, by passing -1 for the others).
 *   rope_cos, rope_sin : nullable fp16 [rope_len, D/2] tables; when given,
 *               each key row is rotated at its own position as in
 *               fa_paged_kv_append_rope (D % 16 == 0).
 * The caller updates seqlen (the reference sets seqlen[b] to at least
 * max_t positions[b, t] + 1, engine/llama_tp.py:88-91).
 */
int fa_paged_kv_scatter(void* k_pages, void* v_pages, const void* k_new, const void* v_new,
                        int B, int Hk, int T, int D, int NB, int P, int page_size,
                        const int32_t* positions, const int32_t* block_table, int max_blocks,
                        const void* rope_cos, const void* rope_sin, int rope_len,
                        void* stream);

/*
 * One decode step: the append of one new token per sequence and the paged
 * attention over the pages that hold it, in one call. Replaces the pair of
 * calls the reference's decode step makes, cache.append (engine/llama_tp.py:
 * 65-78 -> _ext.paged_kv_append, csrc/ext.cpp:70-89) then flash_attn_paged
 * (engine/llama_tp.py:186-200 -> csrc/ext.cpp:42-68), with the same results:
 * it equals fa_paged_kv_append(_rope) with T = 1 followed by
 * fa_flash_attn_paged(_rope)_fwd (k_offset 0, no q_lens).
 *   k_new, v_new : fp16 [B, Hk, 1, D], written into the pages in place.
 *   advance = 0 : the token of sequence b goes to position start_positions[b]
 *                 (or start_pos); seqlen already counts it.
 *   advance = 1 : it goes to position seqlen[b] (start_pos 0, start_positions
 *                 NULL), the attention sees seqlen[b] + 1 keys, and seqlen[b]
 *                 is advanced by one on the device after the attention (the
 *                 reference's seqlen update after the append, llama_tp.py:77).
 *                 For the decode query at the new token's position, pass
 *                 q_offsets = seqlen (read before the advance).
 *   rope_cos, rope_sin : both NULL, or the rotary tables of
 *                 fa_flash_attn_paged_rope_fwd: K is rotated at its position
 *                 as fa_paged_kv_append_rope does, Q at q_off(b) + i.
 *   workspace : as for fa_flash_attn_paged_fwd (fa_paged_workspace_bytes).
 * With advance = 1, when the attention runs on the decode kernels with at
 * most 32 query rows per KV head (heads_per_kv * M <= 32: single-token
 * decode at the benchmark shapes), the append costs no launch of its own:
 * the new token is every sequence's last key, and the decode kernel takes
 * its row from k_new / v_new (rotated there with rotary tables). The merge
 * kernel, which runs after every page read, writes the row into the pages
 * and advances seqlen. Other calls run the append kernel, then the
 * attention (then the advance). The results equal the two calls' as long as
 * no sequence reads a page row that another sequence's new token is written
 * to (pages shared between sequences are read-only to both). No counterpart
 * in the reference, which launches the two separately.
 */
int fa_flash_attn_paged_append_fwd(const void* q, void* k_pages, void* v_pages, int32_t* seqlen,
                                   int page_size, const int32_t* head_map, void* o,
                                   int B, int Hq, int M, int D, int NB, int Hk, int P,
                                   int causal, int64_t q_offset, const int32_t* q_offsets,
                                   const int32_t* block_table, int max_blocks, int heads_per_kv,
                                   const void* k_new, const void* v_new, int advance,
                                   int64_t start_pos, const int32_t* start_positions,
                                   const void* rope_cos, const void* rope_sin, int rope_len,
                                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * Single-sequence decode attention over a token-major fp16 KV cache: the
 * cache layout, head mapping and fp32 input/output of the reference's INT8
 * engine decode step (attn_decode, scripts/deepseek_native_engine.sh:562-604,
 * launched at :1077 after kv_store at :1074), run on the paged-decode kernels:
 *   out[h, :] = sum_{j <= t} softmax_j(scale * q[h, :] . K[j, kvh, :]) V[j, kvh, :]
 *   kvh = head_map ? head_map[h] : h % KVH     (the engine's mapping, :568)
 *   q, out           : fp32 [H, Dh]
 *   k_cache, v_cache : fp16 [>= t + 1, KVH, Dh]; row j of KV head kvh at
 *                      element j*KVH*Dh + kvh*Dh (the engine's Kc/Vc, :553-559)
 * Precision (the engine computes q . k in fp32, :573-577): each query row is
 * scaled by 2^-e (e = 0 unless max|q| >= 2^15, so q beyond the fp16 range
 * does not overflow) and split into fp16 parts q_hi + q_lo, both multiplied
 * by K on the matrix cores with fp32 accumulation. The scores then carry q to
 * about 2^-22 relative (against 2^-11 for q rounded to fp16, which at logits
 * of 30-70 already exceeds the 2e-3 + 1e-2|ref| bar). Softmax and the output
 * accumulate in fp32; the softmax weights enter the P.V product as fp16
 * (2^-11 relative each). A head_map entry outside [0, KVH) yields NaN rows.
 * heads_per_kv: with a head_map, the most heads it sends to one KV head
 * (<= 0: H); ignored without one (the engine's map: ceil(H / KVH)). A map
 * that sends more heads to a KV head breaks the bound: the heads past it get
 * NaN rows, or correct ones where their segment's slot has room (with an
 * even KVH and a bound of at most 8, a segment serves KV heads 2j and 2j + 1
 * and holds 2 * heads_per_kv rows).
 * workspace: fa_decode_token_major_workspace_bytes(H, KVH, Dh, t_max,
 * heads_per_kv) bytes for any t <= t_max (0 when the shape is unsupported);
 * heads_per_kv = ceil(H / KVH) covers the engine's map.
 */
int fa_decode_token_major(float* out, const float* q, const void* k_cache, const void* v_cache,
                          int t, int H, int KVH, int Dh, float scale, const int32_t* head_map,
                          int heads_per_kv, void* workspace, size_t workspace_bytes,
                          void* stream);

size_t fa_decode_token_major_workspace_bytes(int H, int KVH, int Dh, int t_max,
                                             int heads_per_kv);

/* Message of the last failed call on this thread ("" if none). */
const char* fa_last_error(void);

/* FA_ABI_VERSION of the loaded library. */
int fa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FA_MI355X_H */
