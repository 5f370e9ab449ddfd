/*
 * threadcut_hip.h — C ABI of the MI355X (gfx950) decode hot path of threadcut.
 *
 * Three operations, each a hand-written HIP kernel (or kernel pair):
 *   - split-KV GQA flash-decode: a partial online-softmax kernel and a separate
 *     log-sum-exp combine kernel;
 *   - the RoPE delta-shift of post-RoPE keys (new output buffer);
 *   - the in-place suffix splice A.B.C -> A.C of every layer of a KV cache,
 *     fused gather + rotate + store, one launch for all layers.
 *
 * Conventions (all entry points):
 *   - Every pointer argument named *_dev is device memory owned by the caller;
 *     the library allocates no device memory and keeps no per-call state.
 *   - Tensors are described by a base pointer plus element strides. The last
 *     (head_dim) dimension must be contiguous, every base pointer 16-byte
 *     aligned and every stride a multiple of 8 elements (128-bit accesses).
 *   - Element type: fp16 (TC_DTYPE_F16) or bf16 (TC_DTYPE_BF16); head_dim 128.
 *   - `stream` is a hipStream_t (NULL = default stream). Calls only enqueue
 *     work; none synchronizes the host.
 *   - Return value: TC_OK (0) or a TC_ERR_* code. Arguments are validated on
 *     the host before anything is enqueued; tc_last_error() then holds a
 *     message for the calling thread. No entry point aborts the process.
 */
#ifndef THREADCUT_HIP_H
#define THREADCUT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  TC_OK = 0,
  TC_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative size, bad split */
  TC_ERR_UNSUPPORTED = 2,      /* head_dim / group / dtype outside the kernels */
  TC_ERR_ALIGNMENT = 3,        /* base or stride not 16-byte aligned */
  TC_ERR_WORKSPACE = 4,        /* workspace smaller than tc_decode_workspace_bytes */
  TC_ERR_HIP = 5               /* a HIP runtime call failed (message has details) */
};

enum { TC_DTYPE_F16 = 0, TC_DTYPE_BF16 = 1 };

/* Largest number of KV splits one decode call may use. */
#define TC_MAX_SPLITS 4096

/* Decode of caches up to this many tokens with one length for the batch (no
 * per-sequence lengths; not paged, no fused append) runs the partial pass in
 * two-wave work-groups over the same split plan. The tile dealing of
 * tc_decode_partial_interleaved follows the same rule: 16-token tile t goes to
 * split (t / w) % num_splits, w = 2 for such a cache, else 4. */
#define TC_DECODE_SHORT_TOKENS 2048

/* ------------------------------------------------------------------------ */
/* Library information                                                       */
/* ------------------------------------------------------------------------ */

/* Static description of a TC_* code. Never NULL. */
const char* tc_strerror(int code);

/* Message of the last failed call on the calling thread ("" if none). */
const char* tc_last_error(void);

/* ABI version; bumped on any signature change. */
int tc_abi_version(void);

/* ------------------------------------------------------------------------ */
/* Split-KV GQA flash-decode                                                 */
/*                                                                           */
/* Replaces threadcut/flash_decode.py:57-69 (decode_attention: the Triton    */
/* `_partial` launch at :64-67 and the torch softmax(lse)-weighted merge at  */
/* :68-69) and the decode branch of threadcut/attention.py:35-42.            */
/*                                                                           */
/* Shapes: q [B, Hkv, G, D] (the G query heads of KV head h are rows         */
/* h*G .. h*G+G-1 of the model's query heads); k, v [B, Hkv, N, D] where N   */
/* is the buffer's token capacity; lens[b] (optional) is the number of valid */
/* tokens of sequence b, otherwise every sequence has n_tokens tokens. The   */
/* output is [B, Hkv, G, D] with element strides out_strides, in the input   */
/* dtype, fp32 accumulation throughout.                                      */
/* ------------------------------------------------------------------------ */

/* Number of KV splits S a call with these sizes uses (a negative value is
 * -TC_ERR_*). split_tokens <= 0 lets the library choose S so that the
 * B*Hkv*S work-groups match the device's compute units (more of them when
 * `ragged`, i.e. when per-sequence lengths are passed); a positive value is a
 * split length in tokens, rounded up to the kernel's granule (64), as the
 * reference's `split` (threadcut/flash_decode.py:57,61). Host-only; needs no
 * GPU when split_tokens > 0. */
int tc_decode_num_splits(int batch, int kv_heads, int64_t max_tokens, int split_tokens, int ragged);

/* Tokens per split of the same plan (S * tokens >= max_tokens). */
int tc_decode_split_tokens(int batch, int kv_heads, int64_t max_tokens, int split_tokens, int ragged);

/* Bytes of device workspace for num_splits splits: fp32 partial outputs
 * [B, Hkv, S, G, D] followed by fp32 partial log-sum-exps [B, Hkv, S, G]. */
size_t tc_decode_workspace_bytes(int batch, int kv_heads, int group, int head_dim, int num_splits);

/* Partial pass only: writes o_part [B,Hkv,S,G,D] and lse_part [B,Hkv,S,G]
 * (natural log, -inf for a split without tokens). Equivalent of the Triton
 * `_partial` kernel, threadcut/flash_decode.py:21-54. */
int tc_decode_partial(const void* q_dev, const int64_t q_strides[3],
                      const void* k_dev, const int64_t k_strides[3],
                      const void* v_dev, const int64_t v_strides[3],
                      const int32_t* lens_dev, int64_t n_tokens,
                      int batch, int kv_heads, int group, int head_dim, int dtype,
                      float scale, int split_tokens, int num_splits,
                      float* o_part_dev, float* lse_part_dev, void* stream);

/* The partial pass of tc_decode_attention: the same kernel and outputs as
 * tc_decode_partial, but the S splits share each head's 16-token tiles
 * round-robin (split s takes the tiles of waves ws..ws+w-1 in every round of
 * wS tiles; w = 4, or 2 for a cache of at most TC_DECODE_SHORT_TOKENS tokens
 * without lens_dev) instead of owning contiguous slices, so the loads in flight stay
 * adjacent in HBM. A split's partial is the softmax over its own tiles, and
 * tc_decode_combine merges the S partials into the same output as with
 * contiguous slices. For callers that merge partials themselves (for example
 * after exchanging them between GPUs that hold different token ranges), and
 * for timing the pass alone. Same arguments as tc_decode_partial. */
int tc_decode_partial_interleaved(const void* q_dev, const int64_t q_strides[3],
                                  const void* k_dev, const int64_t k_strides[3],
                                  const void* v_dev, const int64_t v_strides[3],
                                  const int32_t* lens_dev, int64_t n_tokens,
                                  int batch, int kv_heads, int group, int head_dim, int dtype,
                                  float scale, int split_tokens, int num_splits,
                                  float* o_part_dev, float* lse_part_dev, void* stream);

/* Combine pass only: out[b,h,g,:] = sum_s softmax_s(lse)[s] * o_part[b,h,s,g,:],
 * cast to dtype (round to nearest even). All-(-inf) lse (no tokens) gives 0.
 * Equivalent of threadcut/flash_decode.py:68-69. */
int tc_decode_combine(const float* o_part_dev, const float* lse_part_dev,
                      int batch, int kv_heads, int group, int head_dim, int num_splits,
                      void* out_dev, const int64_t out_strides[3], int dtype, void* stream);

/* Both passes. workspace_dev must hold tc_decode_workspace_bytes(...) bytes
 * for the split count tc_decode_num_splits(batch, kv_heads, n_tokens,
 * split_tokens, lens_dev != NULL). Lengths past n_tokens are clamped to it.
 * Here the splits are internal, so each takes every S-th 16-token tile of a
 * head (the loads in flight stay adjacent in HBM); the merged output is the
 * same as with contiguous slices. */
int tc_decode_attention(const void* q_dev, const int64_t q_strides[3],
                        const void* k_dev, const int64_t k_strides[3],
                        const void* v_dev, const int64_t v_strides[3],
                        const int32_t* lens_dev, int64_t n_tokens,
                        int batch, int kv_heads, int group, int head_dim, int dtype,
                        float scale, int split_tokens,
                        void* workspace_dev, size_t workspace_bytes,
                        void* out_dev, const int64_t out_strides[3], void* stream);

/* Bytes of the static scratch array of tc_decode_attention_noalloc (per GPU). */
#define TC_DECODE_SCRATCH_BYTES (8u << 20)

/* tc_decode_attention without a workspace. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops that forbid hipMalloc). The split partials go to a
 * static device array of TC_DECODE_SCRATCH_BYTES that each GPU holds until
 * the process ends; the only runtime call besides the two kernel launches is
 * a lookup of that array's address at the first call on a device. A call
 * whose plan needs more than the array (tc_decode_workspace_bytes(...) >
 * TC_DECODE_SCRATCH_BYTES) returns TC_ERR_WORKSPACE and enqueues nothing.
 * The tensors must be on the current device. Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU (other streams, unordered host
 * threads) race and give wrong results; calls ordered on one stream do not.
 * Nothing in the array needs clearing: the partial pass writes every slot the
 * combine pass reads. */
int tc_decode_attention_noalloc(const void* q_dev, const int64_t q_strides[3],
                                const void* k_dev, const int64_t k_strides[3],
                                const void* v_dev, const int64_t v_strides[3],
                                const int32_t* lens_dev, int64_t n_tokens,
                                int batch, int kv_heads, int group, int head_dim, int dtype,
                                float scale, int split_tokens,
                                void* out_dev, const int64_t out_strides[3], void* stream);

/* Append-and-attend for one decode step. The new token's K/V rows k_new /
 * v_new [B, Hkv, D] (element strides (batch, head), last dim contiguous) are
 * written to row n_tokens - 1 of k_cache / v_cache, and the query attends over
 * all n_tokens as tc_decode_attention does: the first n_tokens - 1 from the
 * cache, the last straight from k_new / v_new (so no row is read while it is
 * written). Workspace as tc_decode_attention(..., ragged = 0). This replaces
 * GrowingLayer.update's two strided copies per layer per token
 * (threadcut/kv.py:68-77) together with the decode attention call; the
 * reference has no fused counterpart. */
int tc_decode_append_attention(const void* q_dev, const int64_t q_strides[3],
                               void* k_cache_dev, const int64_t k_strides[3],
                               void* v_cache_dev, const int64_t v_strides[3],
                               const void* k_new_dev, const int64_t k_new_strides[2],
                               const void* v_new_dev, const int64_t v_new_strides[2],
                               int64_t n_tokens, int batch, int kv_heads, int group, int head_dim,
                               int dtype, float scale, int split_tokens,
                               void* workspace_dev, size_t workspace_bytes,
                               void* out_dev, const int64_t out_strides[3], void* stream);

/* tc_decode_append_attention with the append position on the device, so a
 * captured HIP graph of the decode step replays correctly while the cache
 * grows: for sequence b the new token's K/V row is written to row pos[b] of
 * k_cache / v_cache ([B, Hkv, capacity, D] buffers) and the query attends rows
 * [0, pos[b]] (pos[b] cached tokens, then the new one). pos[b] is clamped to
 * [0, capacity - 1]; the caller advances pos (e.g. a kernel in the same graph)
 * and stops before the buffers are full. The split plan and workspace are
 * those of tc_decode_attention(..., n_tokens = capacity, lens = NULL). This is
 * the device-side form of GrowingLayer.update + decode attention
 * (threadcut/kv.py:68-77, threadcut/attention.py:35-39) that the engine's
 * per-token loop (threadcut/engine.py:88-95) needs for graph capture; the
 * reference has no counterpart. */
int tc_decode_append_attention_at(const void* q_dev, const int64_t q_strides[3],
                                  void* k_cache_dev, const int64_t k_strides[3],
                                  void* v_cache_dev, const int64_t v_strides[3],
                                  const void* k_new_dev, const int64_t k_new_strides[2],
                                  const void* v_new_dev, const int64_t v_new_strides[2],
                                  const int32_t* pos_dev, int64_t capacity,
                                  int batch, int kv_heads, int group, int head_dim, int dtype,
                                  float scale, int split_tokens,
                                  void* workspace_dev, size_t workspace_bytes,
                                  void* out_dev, const int64_t out_strides[3], void* stream);

/* Decode over a paged cache. k_pool_dev / v_pool_dev are page pools
 * [num_pages, kv_heads, page_tokens, head_dim] with element strides
 * pool_strides = (page, head, token), shared by K and V. Sequence b attends
 * to the keys of its tiles tile_table_dev[(b * max_tiles + i) * 4 ..],
 * i < tiles_dev[b] (clamped to [0, max_tiles]): int32 {page, first slot,
 * rows, 0}, rows <= 16 consecutive slots of one page. An entry whose page is
 * outside [0, num_pages), whose rows are outside [0, 16] or whose slots run
 * past page_tokens counts as empty. Attention over a set of keys does not
 * depend on their order, so the tiles of a pruned sequence need no
 * compaction. Workspace as tc_decode_attention(..., n_tokens =
 * 16 * max_tiles, ragged = batch > 1). This is decode_attention
 * (threadcut/flash_decode.py:57-69) over the paged KV with slot reuse that
 * the threadcut repository's README.md:141-144 names as the next step. */
int tc_decode_paged_attention(const void* q_dev, const int64_t q_strides[3],
                              const void* k_pool_dev, const void* v_pool_dev,
                              const int64_t pool_strides[3], int num_pages, int page_tokens,
                              const int32_t* tile_table_dev, const int32_t* tiles_dev,
                              int64_t max_tiles, int batch, int kv_heads, int group,
                              int head_dim, int dtype, float scale, int split_tokens,
                              void* workspace_dev, size_t workspace_bytes,
                              void* out_dev, const int64_t out_strides[3], void* stream);

/* One paged decode step with the cache append fused in, the paged form of
 * tc_decode_append_attention. The caller has already reserved each
 * sequence's slot for the new token, so the tile table includes it as the
 * last row of the sequence's last tile (tiles_dev[b] >= 1). The query attends
 * the other keys of the table from the pools and the new token straight from
 * k_new / v_new ([B, Hkv, D], element strides (batch, head)); wave 0 of split
 * 0 writes the new K/V row into its slot, which no other wave reads. A last
 * tile entry that is out of range writes nothing. Workspace as
 * tc_decode_paged_attention. This replaces GrowingLayer.update's two copies
 * per layer (threadcut/kv.py:68-77) with the decode call for a paged cache;
 * the reference has no counterpart. */
int tc_decode_paged_append_attention(const void* q_dev, const int64_t q_strides[3],
                                     void* k_pool_dev, void* v_pool_dev,
                                     const int64_t pool_strides[3], int num_pages, int page_tokens,
                                     const int32_t* tile_table_dev, const int32_t* tiles_dev,
                                     int64_t max_tiles, const void* k_new_dev,
                                     const int64_t k_new_strides[2], const void* v_new_dev,
                                     const int64_t v_new_strides[2], int batch, int kv_heads,
                                     int group, int head_dim, int dtype, float scale,
                                     int split_tokens, void* workspace_dev, size_t workspace_bytes,
                                     void* out_dev, const int64_t out_strides[3], void* stream);

/* The same step with the sequence lengths on the device, so that one captured
 * HIP graph serves every step (the per-token loop of threadcut/engine.py:88-95
 * over a paged cache; no counterpart in the reference). Sequence b holds
 * lens_dev[b] tokens before the step; its new token goes to logical position
 * lens_dev[b], whose row sits tok_off_dev[b * tok_pitch + lens_dev[b]] bytes
 * into the head slab of the pools (an offset outside the pool writes
 * nothing). A sequence whose lens_dev[b] is tok_pitch or more has no offset
 * row for its new token: nothing is written for it, and the call still
 * attends its cached rows below lens_dev[b] and the new token. The tile table
 * covers slots reserved ahead: each entry's 4th word is its first logical
 * position, and only rows below lens_dev[b] are read.
 * The split plan depends on max_tiles only, so the caller advances lens_dev
 * between steps (on the device, inside the graph) and nothing else changes.
 * Pools must be under 2 GiB (32-bit offsets). Workspace as
 * tc_decode_paged_attention. */
int tc_decode_paged_append_attention_at(const void* q_dev, const int64_t q_strides[3],
                                        void* k_pool_dev, void* v_pool_dev,
                                        const int64_t pool_strides[3], int num_pages, int page_tokens,
                                        const int32_t* tile_table_dev, const int32_t* tiles_dev,
                                        int64_t max_tiles, const int32_t* tok_off_dev, int64_t tok_pitch,
                                        const int32_t* lens_dev, const void* k_new_dev,
                                        const int64_t k_new_strides[2], const void* v_new_dev,
                                        const int64_t v_new_strides[2], int batch, int kv_heads,
                                        int group, int head_dim, int dtype, float scale,
                                        int split_tokens, void* workspace_dev, size_t workspace_bytes,
                                        void* out_dev, const int64_t out_strides[3], void* stream);

/* ------------------------------------------------------------------------ */
/* RoPE delta-shift and suffix splice                                        */
/*                                                                           */
/* cos_sin_host: 2*(head_dim/2) fp32 values on the HOST, cos(angle_i) then   */
/* sin(angle_i) for i < head_dim/2, angle_i = delta * inv_freq_i, exactly as */
/* threadcut/kv.py:22-23 builds `emb` (emb = cat(angle, angle), so the upper */
/* half reuses the same values). The table travels in the kernel arguments.  */
/* Per element: out = fp16(fl(k*cos) + fl(rotate_half(k)*sin)), no fused     */
/* multiply-add, matching threadcut/kv.py:25 op for op.                      */
/* ------------------------------------------------------------------------ */

/* keys [B, H, T, D] (strides src_strides) -> out [B, H, T, D] (strides
 * dst_strides). out may not alias keys. Replaces threadcut/kv.py:20-25
 * (shift_keys). */
int tc_shift_keys(const void* keys_dev, const int64_t src_strides[3],
                  void* out_dev, const int64_t dst_strides[3],
                  int batch, int heads, int64_t tokens, int head_dim, int dtype,
                  const float* cos_sin_host, void* stream);

/* In place, for every layer l < num_layers, every batch row and head:
 *   K[a + t] <- shift(K[c0 + t]),  V[a + t] <- V[c0 + t]   for t < c
 * with the memmove semantics of the reference's clone-then-write (sources
 * are read before they are overwritten, also when c0 - a < c). Rows outside
 * [a, a+c) are not touched. k_layers_host / v_layers_host are HOST arrays of
 * num_layers device pointers to [B, H, cap, D] buffers that share `strides`.
 * c0 == a (no gap) or c == 0 enqueues nothing. cos_sin_host may be NULL
 * only then. Replaces threadcut/kv.py:28-33 + :83-92 (splice over
 * GrowingLayer.splice, 36 per-layer torch op chains) with one launch. */
int tc_splice_rope(void* const* k_layers_host, void* const* v_layers_host, int num_layers,
                   const int64_t strides[3], int batch, int heads, int64_t capacity,
                   int head_dim, int dtype, int64_t a, int64_t c0, int64_t c,
                   const float* cos_sin_host, void* stream);

/* Out of place: for every layer, rows [0, a) of src are copied to rows
 * [0, a) of dst, and rows [c0, c0+c) of src to rows [a, a+c) of dst, keys
 * shifted. This is the index_select branch of threadcut/kv.py:34-41 for
 * caches whose layers are not preallocated buffers. dst must not alias src.
 * a + c == 0 keeps nothing: no pointer is needed and nothing is enqueued. */
int tc_splice_copy(void* const* k_src_host, void* const* v_src_host,
                   const int64_t src_strides[3], int64_t src_tokens,
                   void* const* k_dst_host, void* const* v_dst_host,
                   const int64_t dst_strides[3], int num_layers,
                   int batch, int heads, int head_dim, int dtype,
                   int64_t a, int64_t c0, int64_t c,
                   const float* cos_sin_host, void* stream);

/* The splice of a paged cache: the keys of the kept suffix are rotated in
 * place by the angle table cos_sin_host (the shift of tc_shift_keys); V is
 * not touched. For every layer's K pool (k_pools_host: HOST array of
 * num_layers device pointers to pools laid out as in
 * tc_decode_paged_attention) and every head, the rows of the num_tiles
 * entries of tiles_dev (int32 {page, first slot, rows, 0}, the tile format of
 * tc_decode_paged_attention) are rotated. Entries must not overlap (a row
 * listed twice is rotated twice); invalid entries are skipped. With pages,
 * dropping the pruned span frees its pages, so this replaces the suffix move
 * of threadcut/kv.py:28-41,83-92, as the threadcut repository's README.md:141-144 proposes. */
int tc_paged_rotate_keys(void* const* k_pools_host, int num_layers, const int64_t pool_strides[3],
                         int num_pages, int page_tokens, const int32_t* tiles_dev,
                         int64_t num_tiles, int kv_heads, int head_dim, int dtype,
                         const float* cos_sin_host, void* stream);

/* ------------------------------------------------------------------------ */
/* Prefill attention                                                         */
/* ------------------------------------------------------------------------ */

/* The prefill branch of threadcut/attention.py:43-46 without expanding the
 * KV heads (repeat_kv, attention.py:25-27): for query token t of every
 * query head hq = h*g + i (g = q_heads / kv_heads),
 *   out[b, t, hq, :] = softmax_j(q[b, hq, t]·k[b, h, j]ᵀ·scale + mask)·v[b, h, j]
 * over keys j < n_tokens, fp32 softmax and accumulation. The query tokens sit
 * at positions n_tokens - q_len + t. Masking is one of
 *   - mask != NULL: boolean [mb, q_len, n_tokens] bytes (1 = attend) with
 *     element strides mask_strides (batch stride 0 broadcasts one mask over
 *     the batch); causal must be 0. mask_tiles, if not NULL, is the map
 *     tc_prefill_mask_tiles built for this mask and these sizes (it lets the
 *     kernel skip fully masked 64-key tiles and test no element of fully
 *     visible ones); NULL tests every element;
 *   - causal != 0: key j visible to token t iff j <= n_tokens - q_len + t
 *     (SDPA's is_causal when q_len == n_tokens);
 *   - neither: every key visible.
 * A query row with no visible key gets zeros. q [b, hq, q_len, d] and k/v
 * [b, hkv, n_tokens, d] with element strides {batch, head, token} and a
 * contiguous last dim; out [b, q_len, hq, d] with strides {batch, token,
 * head}. head_dim must be 128, g one of 1, 2, 4, 8. num_splits <= 0 picks
 * the key split count (tc_prefill_num_splits); the workspace must hold
 * tc_prefill_workspace_bytes for the count used (none for one split). */
int tc_prefill_attention(const void* q, const int64_t q_strides[3],
                         const void* k, const int64_t k_strides[3],
                         const void* v, const int64_t v_strides[3],
                         const uint8_t* mask, const int64_t mask_strides[3],
                         const uint8_t* mask_tiles, size_t mask_tiles_bytes, int causal,
                         int64_t q_len, int64_t n_tokens, int batch, int q_heads, int kv_heads,
                         int head_dim, int dtype, float scale,
                         int num_splits, void* workspace, size_t workspace_bytes,
                         void* out, const int64_t out_strides[3], void* stream);

/* tc_prefill_attention over a paged cache: the prefill branch of
 * threadcut/attention.py:43-46 for a cache kept in page pools (the layout the
 * reference's README.md:141-144 proposes). K and V are pools [pages, Hkv, P,
 * D] with element strides pool_strides {page, head, slot}; sequence b's
 * logical key t (t < n_tokens) is the row tok_off_dev[b * tok_pitch + t]
 * bytes into a head's slab (the same offset in K and V). Keys keep their
 * logical order, so masks, is_causal and the tile map mean what they mean
 * for tc_prefill_attention, whose other arguments this takes unchanged.
 * Pools must be under 2 GiB (32-bit offsets); an offset outside the pool
 * reads zeros. */
int tc_prefill_paged_attention(const void* q, const int64_t q_strides[3],
                               const void* k_pool, const void* v_pool, const int64_t pool_strides[3],
                               int num_pages, const int32_t* tok_off, int64_t tok_pitch,
                               const uint8_t* mask, const int64_t mask_strides[3],
                               const uint8_t* mask_tiles, size_t mask_tiles_bytes, int causal,
                               int64_t q_len, int64_t n_tokens, int batch, int q_heads, int kv_heads,
                               int head_dim, int dtype, float scale,
                               int num_splits, void* workspace, size_t workspace_bytes,
                               void* out, const int64_t out_strides[3], void* stream);

/* Key splits tc_prefill_attention uses with num_splits <= 0 (a negative value
 * is -TC_ERR_*): 1 when the query blocks (128 rows of one KV head each) give
 * every compute unit two work-groups, else enough splits of the keys to do
 * so, merged by a log-sum-exp combine pass. A short chunk on top of a long
 * cache (the engine's prefill after a splice) is the case this covers. */
int tc_prefill_num_splits(int batch, int64_t q_len, int64_t n_tokens, int q_heads, int kv_heads);

/* Workspace bytes of a call with num_splits splits (0 for one split): fp32
 * partial outputs [b, splits, q_len, hq, d] then log-sum-exps [b, splits, q_len, hq]. */
size_t tc_prefill_workspace_bytes(int batch, int64_t q_len, int q_heads, int num_splits);

/* Bytes of the tile map of a mask with mask_batch distinct batch entries
 * (1 for a broadcast mask); 0 for invalid sizes. */
size_t tc_prefill_tiles_bytes(int64_t q_len, int64_t n_tokens, int mask_batch, int q_heads, int kv_heads);

/* Classifies every (query block of 128/g tokens, 64-key tile) of a boolean
 * mask as skip / full / causal (exactly key <= n_tokens - q_len + token, the
 * mask of a chunk on top of a cache) / mixed into `tiles` for
 * tc_prefill_attention. One
 * read of the mask; the map stays valid while the mask is unchanged, so the
 * layers of one forward pass share it. Part of the prefill branch above
 * (threadcut/attention.py:43-46); the reference has no separate step. */
int tc_prefill_mask_tiles(const uint8_t* mask, const int64_t mask_strides[3], int mask_batch,
                          int64_t q_len, int64_t n_tokens, int q_heads, int kv_heads,
                          uint8_t* tiles, size_t tiles_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Request split (host code, no GPU)                                         */
/* ------------------------------------------------------------------------ */

/* Split(a, c0, c) of `fresh` against `cached` by the rule of
 * threadcut/match.py:33-48 (longest common prefix capped at n_fresh - 1; the
 * longest run of fresh[a:] that also starts in cached[a+1:] from a
 * min_suffix-token anchor, first longest wins, capped at len(fresh[a:]) - 1;
 * (a, a, 0) when suffix is 0 or too short). out = {a, c0, c}. The anchor
 * search is a rolling hash, linear in n_cached plus the verified hits. */
int tc_match_split(const int64_t* cached, int64_t n_cached, const int64_t* fresh, int64_t n_fresh,
                   int64_t min_suffix, int suffix, int64_t out[3]);

/* ------------------------------------------------------------------------ */
/* Page tables of the paged cache (host code, no GPU)                        */
/* ------------------------------------------------------------------------ */

/* The paged cache is this library's own (threadcut/README.md:141-144 proposes
 * it; threadcut/kv.py:28-41,83-92 is the move it replaces): no reference
 * function has these signatures. A sequence is a list of fragments, rows of
 * int64 {page, first slot, count} in logical order (count >= 1 consecutive
 * slots of one page). Each function takes the pool's page size, page_tokens,
 * and refuses (TC_ERR_INVALID_ARGUMENT) a list with a fragment that runs past
 * its page (first slot + count > page_tokens), a negative page or slot, or an
 * empty fragment.
 *
 * Tile entries {page, first slot, rows, logical start} of the fragments, each
 * cut at multiples of 16 slots (the tile table of tc_decode_paged_attention,
 * the tile list of tc_paged_rotate_keys); the first fragment starts at
 * logical position first_pos. Returns the number of entries and writes them
 * only when max_tiles is at least that (tiles may be NULL to ask), or
 * -TC_ERR_INVALID_ARGUMENT for a malformed fragment. */
int64_t tc_page_tiles(const int64_t* frags, int64_t num_frags, int64_t page_tokens, int64_t first_pos, int32_t* tiles,
                      int64_t max_tiles);

/* Prune of one sequence: keep logical tokens [0, a) and [c0, c0 + c). kept
 * (room for num_frags + 1 rows) receives the new fragment list, the two kept
 * ranges joined (their pieces merge when they are adjacent slots of one
 * page); suffix (num_frags rows) the fragments of [c0, c0 + c) alone; freed
 * (num_frags entries) the pages no kept fragment uses, ascending.
 * counts = {kept rows, suffix rows, freed pages}. */
int tc_page_prune(const int64_t* frags, int64_t num_frags, int64_t page_tokens, int64_t a, int64_t c0, int64_t c,
                  int64_t* kept, int64_t* suffix, int64_t* freed, int64_t counts[3]);

/* Byte offset of every logical token's row in a head slab of the pools,
 * page * page_bytes + slot * slot_bytes, for the tokens of the fragments, and
 * INT32_MIN (past every buffer range) up to pitch (the per-token offsets of
 * tc_prefill_paged_attention and tc_decode_paged_append_attention_at).
 * Returns the token count, or -TC_ERR_INVALID_ARGUMENT when it exceeds pitch,
 * a fragment is malformed or an offset passes 2^31 - 1. */
int64_t tc_page_token_offsets(const int64_t* frags, int64_t num_frags, int64_t page_tokens, int64_t page_bytes,
                              int64_t slot_bytes, int32_t* out, int64_t pitch);

#ifdef __cplusplus
}
#endif

#endif /* THREADCUT_HIP_H */
