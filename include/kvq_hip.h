/* SPDX-License-Identifier: Apache-2.0
 *
 * kvq_hip.h -- C ABI of libkvq_hip.so, the MI355X (gfx950) kernels of the
 * quantized-KV hot path.
 *
 * Conventions
 *   - Every pointer is a device pointer owned by the caller (the Python layer
 *     allocates through torch); the library never allocates.  Workspaces are
 *     passed in and their sizes are given by the *_workspace_bytes helpers.
 *   - Sizes are int64_t, geometry is int; dtype and index-width arguments use
 *     the enums below.  `stream` is a hipStream_t passed as void*.
 *   - Return 0 on success; KVQ_ERR_* (< 0) for rejected arguments; a positive
 *     hipError_t if the launch failed.  Nothing is launched when an argument
 *     is rejected.
 *   - Calls are asynchronous on `stream`, run entirely on it, and are
 *     thread-safe.  The only state the library keeps is per device: cached
 *     device limits (LDS per workgroup, resident workgroups per kernel),
 *     filled on first use, and the static scratch array of
 *     kvq_kivi_decode_attn_noalloc (with its device address).
 *
 * Reference paths are relative to /root/reference with
 * pkg/ = src/vllm_ascend_quantized_kv_cache/; each entry point names the
 * reference interface it replaces.
 */
#ifndef KVQ_HIP_H_
#define KVQ_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  KVQ_DTYPE_F32 = 0,
  KVQ_DTYPE_F16 = 1,
  KVQ_DTYPE_BF16 = 2,
};

enum {
  KVQ_INDEX_I32 = 0,
  KVQ_INDEX_I64 = 1,
};

enum {
  KVQ_OK = 0,
  KVQ_ERR_INVALID = -1,     /* bad pointer, dtype or size */
  KVQ_ERR_GEOMETRY = -2,    /* geometry the kernels do not support */
  KVQ_ERR_SCRATCH = -3,     /* work larger than the library's static scratch */
  KVQ_ERR_CAPACITY = -4,    /* output arrays too small for the plan */
};

/* Decode work plans (kvq_plan_kivi_decode). */
enum {
  KVQ_PLAN_DEFAULT = 0,       /* pieces when the work fills the chip once, else paired splits */
  KVQ_PLAN_PIECES = 1,        /* cost-balanced pieces (one or more rounds) */
  KVQ_PLAN_SPLIT = 2,         /* int4 ranges every split_tokens positions */
  KVQ_PLAN_SPLIT_PAIRED = 3,  /* as SPLIT, each range as an even/odd-chunk pair */
};

/* Size of the static device scratch behind kvq_kivi_decode_attn_noalloc. */
#define KVQ_DECODE_SCRATCH_BYTES (32ll << 20)

/* ABI version: bumped whenever a signature below changes. */
int kvq_abi_version(void);

/* ---- KIVI INT4 ---------------------------------------------------------- */

/* Key pack: token groups of `group_size` tokens -> k_quant [NB,KVH,D,Bs/8]
 * int32 words (lane = block offset % 8), k_scale/k_mn [NB,KVH,D,Bs/G] fp32.
 * Replaces kivi_pack_key_cache (pkg/ops/triton/kivi_pack.py:287-348) and its
 * kernel (:134-226).
 * Token t of the batch reads source row r = src_index ? src_index[t] : t from
 * src_a (rows [0, n_a)) or src_b (rows >= n_a, index r - n_a); rows are
 * [KVH, D] contiguous of `src_dtype`.  num_tokens % group_size == 0; each
 * group's slots must be contiguous, group aligned and inside one block (the
 * caller validates); a group whose first slot is negative is skipped. */
int kvq_kivi_pack_key(const void* src_a, int64_t n_a, const void* src_b,
                      const int64_t* src_index, int src_dtype,
                      const void* slot_mapping, int slot_index_type, int64_t num_tokens,
                      int num_kv_heads, int head_size, int group_size, int block_size,
                      int32_t* k_quant, float* k_scale, float* k_mn, void* stream);

/* Value pack: per (token, head, head-dim group) -> v_quant [NB,Bs,KVH,D/8]
 * int32 (lane = dim % 8), v_scale/v_mn [NB,Bs,KVH,D/G] fp32.  Tokens with a
 * negative slot are skipped.  Source rows as for kvq_kivi_pack_key.
 * Replaces kivi_pack_value_cache (pkg/ops/triton/kivi_pack.py:229-284) and its
 * kernel (:61-131). */
int kvq_kivi_pack_value(const void* src_a, int64_t n_a, const void* src_b,
                        const int64_t* src_index, int src_dtype,
                        const void* slot_mapping, int slot_index_type, int64_t num_tokens,
                        int num_kv_heads, int head_size, int group_size, int block_size,
                        int32_t* v_quant, float* v_scale, float* v_mn, void* stream);

/* Residual-ring write: ring row dst_rows[i] (a row is KVH*D elements of
 * `ring_dtype`, the ring viewed as [rows*ring_len, KVH, D]) takes source row
 * src_rows[i] (identity when NULL) of `src_dtype`, converted with
 * round-to-nearest-even.  Replaces the per-token lane writes of
 * _store_kivi_residual_entries (pkg/methods/kivi_int4/attention_backend.py:
 * 411-462), batched over every token and request of a step. */
int kvq_kivi_ring_write(const void* src, int src_dtype, const int64_t* src_rows,
                        const int64_t* dst_rows, int64_t num_rows, int row_elems,
                        void* ring, int ring_dtype, void* stream);

/* One-launch store of a batch: the key pack, value pack and both sides' ring
 * writes of kvq_kivi_pack_key / kvq_kivi_pack_value / kvq_kivi_ring_write in
 * a single grid.  Replaces the flush-then-append sequence of
 * _store_kivi_residual_entries (pkg/methods/kivi_int4/attention_backend.py:
 * 442-462, with _flush_kivi_residual_prefix) for a whole step.
 * jobs (int64, device): [key pack src | key pack slot | value pack src |
 * value pack slot | key ring src | key ring dst | value ring src | value ring
 * dst] with n_key_pack, n_value_pack, n_key_ring, n_value_ring entries.  Pack
 * sources index [ring rows (ring_rows of them) ; input rows]; ring src are
 * input rows, ring dst ring rows.  Inputs and rings are [rows, KVH, D] of
 * `dtype`.  Precondition: no ring dst is a pack source of the same side (the
 * batch then has no order inside it).  Head size 128, group size 64 or 128,
 * bf16/fp16 only: other geometries return KVQ_ERR_GEOMETRY and the caller
 * uses the separate entry points.  n_key_pack % group_size == 0 with the
 * group rules of kvq_kivi_pack_key. */
int kvq_kivi_store(const void* key_input, const void* value_input, void* ring_k,
                   void* ring_v, int64_t ring_rows, int dtype, int num_kv_heads,
                   int head_size, int group_size, int block_size, const int64_t* jobs,
                   int64_t n_key_pack, int64_t n_value_pack, int64_t n_key_ring,
                   int64_t n_value_ring, int32_t* k_quant, float* k_scale, float* k_mn,
                   int32_t* v_quant, float* v_scale, float* v_mn, void* stream);

/* Paged gather-dequant to dense TND with an optional residual-tail overlay.
 * out_k/out_v are [cu_seqlens[batch], KVH, D] of `out_dtype`; request b owns
 * rows [cu_seqlens[b], cu_seqlens[b+1]).  Negative block ids read block 0 and
 * are masked by the sequence length.  Dequant is q*scale then +mn (two fp32
 * roundings) then a round-to-nearest-even cast.
 * Overlay (ring_k != NULL): ring_meta is int32 [batch, 5] =
 *   {ring_row, k_first_lane, k_tail, v_first_lane, v_tail};
 * the last k_tail rows of request b come from ring_k[ring_row, (k_first_lane
 * + i) % ring_len] (i = 0..k_tail-1), likewise for values; ring tensors are
 * [rows, ring_len, KVH, D] of `ring_dtype`.
 * Replaces kivi_dequant_gather_cache (pkg/ops/kivi_gather.py:36-156) plus the
 * overlay loop of _gather_dequant_kivi_paged_cache
 * (pkg/methods/kivi_int4/attention_backend.py:849-935). */
int kvq_kivi_gather_dequant(const int32_t* k_quant, const float* k_scale, const float* k_mn,
                            const int32_t* v_quant, const float* v_scale, const float* v_mn,
                            int64_t num_blocks, int block_size, int num_kv_heads,
                            int head_size, int group_size,
                            const void* block_table, int block_index_type, int64_t max_blocks,
                            const int64_t* cu_seqlens, int64_t batch,
                            const int32_t* ring_meta, const void* ring_k, const void* ring_v,
                            int ring_dtype, int ring_len,
                            void* out_k, void* out_v, int out_dtype, void* stream);

/* Fused KIVI INT4 decode attention: one query token per request attends to
 * its int4 history (dequantized in registers) and its full-precision residual
 * window, split over a work list and merged with a log-sum-exp combine.
 *   query/out   [batch, num_heads, D] of `q_dtype`
 *   seq_meta    int32 [batch, 8] = {seq_len, k_hist, v_hist, ring_row,
 *               k_first_lane, v_first_lane, first_work, num_work}
 *               positions < k_hist (v_hist) read int4 keys (values); the
 *               others read ring lane (first_lane + p - hist) % ring_len
 *   work        int32 [num_work, 4] = {request, pos_begin, pos_end, kind}
 *               kind 0: both sides int4 over the whole range, pos_begin a
 *                       multiple of 64 (the int4 MFMA kernel's tiles);
 *               kind 1: any mix of sources (the MFMA kernel's tail path, the
 *                       standalone MFMA tail kernel, or the generic kernel
 *                       for geometries neither covers)
 *               kind 2 / 3: as kind 0 (pos_begin a multiple of 64), over
 *                       the even / odd 64-position chunks of the range only.
 *                       A kind-2 item at an even index followed by its
 *                       kind-3 twin run on one XCD at the same time and
 *                       share the range's key lines through its L2.
 *               a request's items are contiguous, from first_work on
 *   pieces      int32 [num_pieces + 1] or NULL: piece k is work items
 *               [pieces[k], pieces[k+1]).  At num_kv_heads 8, D 128,
 *               block_size 128, group_size 64 or 128, at most 16 query
 *               heads per kv head and 16-bit query and ring, two workgroups
 *               per piece (one per half of the kv heads) stream the piece's
 *               kind-0 items page by page, then run its tail items (plan with
 *               split_tokens 128 so that no two pieces share a page).
 *               Elsewhere, where the MFMA kernel runs both kinds, one wave
 *               per (piece, kv head) runs its piece's items in order in a
 *               single pass, so pieces of equal cost end together; else the
 *               pieces are ignored.
 *   workspace   >= kvq_kivi_decode_workspace_bytes(num_work, num_heads, D)
 *   block_table int32 [batch, max_blocks]
 * Replaces the decode branch: _forward_kivi_paged_decode_attention
 * (pkg/methods/kivi_int4/attention_backend.py:1193-1230), i.e. the gather of
 * :849-935 followed by npu_fused_infer_attention_score (TND, sparse_mode 0). */
int64_t kvq_kivi_decode_workspace_bytes(int64_t num_work, int num_heads, int head_size);
int kvq_kivi_decode_attn(const void* query, int q_dtype, int64_t batch, int num_heads,
                         int num_kv_heads, int head_size, float scale,
                         const int32_t* k_quant, const float* k_scale, const float* k_mn,
                         const int32_t* v_quant, const float* v_scale, const float* v_mn,
                         int64_t num_blocks, int block_size, int group_size,
                         const int32_t* block_table, int64_t max_blocks,
                         const int32_t* seq_meta, const int32_t* work, int64_t num_work,
                         const int32_t* pieces, int64_t num_pieces,
                         const void* ring_k, const void* ring_v, int ring_dtype, int ring_len,
                         void* workspace, void* out, void* stream);

/* kvq_kivi_decode_attn without a workspace argument: the split-K partials go
 * to a static device array of KVQ_DECODE_SCRATCH_BYTES (32 MiB) that each GPU
 * the library runs on holds until the process ends; the call allocates
 * nothing (no hipMalloc, no library allocation).  Work lists whose partials
 * (kvq_kivi_decode_workspace_bytes) exceed it return KVQ_ERR_SCRATCH before
 * anything is launched.  The stream must belong to the calling thread's
 * current device.  Every call on one GPU shares that GPU's array and leaves
 * the last call's partials in it: calls that overlap on one GPU (two streams,
 * or two threads) race and must be serialized by the caller.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). */
int kvq_kivi_decode_attn_noalloc(const void* query, int q_dtype, int64_t batch, int num_heads,
                                 int num_kv_heads, int head_size, float scale,
                                 const int32_t* k_quant, const float* k_scale,
                                 const float* k_mn, const int32_t* v_quant,
                                 const float* v_scale, const float* v_mn, int64_t num_blocks,
                                 int block_size, int group_size, const int32_t* block_table,
                                 int64_t max_blocks, const int32_t* seq_meta,
                                 const int32_t* work, int64_t num_work, const int32_t* pieces,
                                 int64_t num_pieces, const void* ring_k, const void* ring_v,
                                 int ring_dtype, int ring_len, void* out, void* stream);

/* Host-side (no GPU call): the work list, and pieces, of kvq_kivi_decode_attn
 * for a batch, written into caller arrays (plain host memory; pinned memory
 * lets the caller copy the plan to the device without a synchronisation).
 *   seqs      int32 [batch, 6] = {seq_len, k_hist, v_hist, ring_row,
 *             k_first_lane, v_first_lane} (the seq_meta columns it fills)
 *   seq_meta  int32 [batch, 8]; work int32 [cap_work, 4];
 *   pieces    int32 [cap_pieces + 1] (KVQ_PLAN_PIECES / DEFAULT)
 *   mode      KVQ_PLAN_*; split_tokens for the SPLIT modes, and for
 *             KVQ_PLAN_PIECES the int4 tile (0 or 64: kind-0 items cut on
 *             64-position bounds; 128: on 128-position bounds, the pages of
 *             the page-streaming decode); tail_cost = the cost of one
 *             residual-window position in int4 positions
 * Returns the number of work items, *num_pieces (0 for split plans), or
 * KVQ_ERR_INVALID / KVQ_ERR_CAPACITY.  Replaces the per-step decode planning
 * a host does before _forward_kivi_paged_decode_attention
 * (pkg/methods/kivi_int4/attention_backend.py:1193-1230): which positions
 * read int4 pages and which the residual window, split over the chip. */
int64_t kvq_plan_kivi_decode(const int32_t* seqs, int64_t batch, int num_kv_heads, int cu_count,
                             int mode, int64_t split_tokens, double tail_cost, int32_t* seq_meta,
                             int32_t* work, int64_t cap_work, int32_t* pieces,
                             int64_t cap_pieces, int64_t* num_pieces);

/* Host checks of one decode step (host arrays, no device access), in one
 * pass: the gather's metadata gate (pkg/ops/kivi_layout.py:205-238: the
 * table covers the longest sequence, live block ids lie in [0, num_blocks))
 * and the window-entry liveness of the residual rows
 * (pkg/methods/kivi_int4/attention_backend.py:813-836: an entry written at
 * position p with slot s is live while p < seq_len and the request's table
 * still holds s's block at column p / block_size).
 *   table int64 [batch, max_blocks]; seq_lens, rows int64 [batch] (ring row
 *   of each request, -1 for none); k_slot, k_pos, v_slot, v_pos int64
 *   [ring_rows, ring_len] (the host mirror of both windows)
 * *kind: 0 (pass), 1 (a live block id < 0), 2 (a live block id >=
 * num_blocks; the return value is the first such request), 3 (the table does
 * not cover the longest sequence).  suspect[i] = 1 when request i's window
 * holds an entry that may no longer be live.  Returns >= 0, or
 * KVQ_ERR_INVALID. */
int64_t kvq_kivi_step_check(const int64_t* table, int64_t batch, int64_t max_blocks,
                            const int64_t* seq_lens, int64_t num_blocks, int64_t block_size,
                            const int64_t* rows, const int64_t* k_slot, const int64_t* k_pos,
                            const int64_t* v_slot, const int64_t* v_pos, int64_t ring_rows,
                            int64_t ring_len, int32_t* suspect, int32_t* kind);

/* kvq_kivi_store with its counts and jobs in one device buffer, sized for
 * capacities: plan (int64, device) = [n_key_pack, n_value_pack, n_key_ring,
 * n_value_ring, key pack src[cap_key_pack], key pack slot[cap_key_pack],
 * value pack src[cap_value_pack], value pack slot[cap_value_pack], key ring
 * src[cap_ring], key ring dst[cap_ring], value ring src[cap_ring], value ring
 * dst[cap_ring]].  The grid covers the capacities and each wave reads the
 * counts, so one launch, captured once in a HIP graph, serves every step
 * whose plan the host copies into the buffer before it runs.  Same
 * preconditions and geometry as kvq_kivi_store.  Replaces, like
 * kvq_kivi_store, a step of _store_kivi_residual_entries
 * (pkg/methods/kivi_int4/attention_backend.py:411-462). */
int kvq_kivi_store_planned(const void* key_input, const void* value_input, void* ring_k,
                           void* ring_v, int64_t ring_rows, int dtype, int num_kv_heads,
                           int head_size, int group_size, int block_size, const int64_t* plan,
                           int64_t cap_key_pack, int64_t cap_value_pack, int64_t cap_ring,
                           int32_t* k_quant, float* k_scale, float* k_mn, int32_t* v_quant,
                           float* v_scale, float* v_mn, void* stream);

/* ---- dense attention ----------------------------------------------------- */

/* Attention over dense TND tensors: query [cu_q[batch], num_heads, D], key and
 * value [cu_k[batch], num_kv_heads, D], out like query, all of `dtype`.
 * Request b's query row i sits at kv position lk_b - lq_b + i; with `causal`
 * keys past it are masked.  GQA maps query head h to kv head
 * h / (num_heads / num_kv_heads).  cu_* are int32 [batch + 1]; max_q_len
 * bounds lq_b.  head_size in {32, 64, 128, 256}; scale > 0.
 * Replaces npu_fused_infer_attention_score with input_layout "TND"
 * (pkg/methods/kivi_int4/attention_backend.py:1248-1262, 1320-1334 and the
 * dense fallback 1341-1392; pkg/methods/int8_dynamic/attention_backend.py:
 * 282-296, 350-364). */
int kvq_prefill_attn(const void* query, const void* key, const void* value, int dtype,
                     const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                     int64_t batch, int64_t max_q_len, int num_heads, int num_kv_heads,
                     int head_size, float scale, int causal, void* out, void* stream);

/* ---- INT8 dynamic per-channel ------------------------------------------- */

/* First-K/V scales in the activation dtype: amax over tokens per (head, dim),
 * clamp_min(1e-12), inv = (1/amax)*127, aq = 1/inv, every step rounded to
 * `dtype` as torch evaluates `127.0 / k_max` (reciprocal then multiply).
 * key/value [num_tokens, KVH*D]; k_inv/v_inv/k_aq/v_aq [KVH*D] of `dtype`;
 * amax_ws: uint32 [2*KVH*D] workspace (zeroed by this call).
 * Replaces _prepare_int8_scales (pkg/methods/int8_dynamic/attention_backend.py:130-150)
 * == Int8DynamicSemantics.calc_scales (pkg/methods/int8_dynamic/semantics.py:49-70). */
int kvq_int8_calc_scales(const void* key, const void* value, int dtype, int64_t num_tokens,
                         int64_t channels, uint32_t* amax_ws, void* k_inv, void* v_inv,
                         void* k_aq, void* v_aq, void* stream);

/* Quantize clamp(round_half_even(x*inv), -128, 127) (product rounded to
 * `dtype`) and scatter by slot into key_cache/value_cache [NB,Bs,KVH,D] int8.
 * Negative slots are padding and skipped.
 * Replaces _quantize_kv_to_runtime_int8 (attention_backend.py:152-171) plus the
 * host reshape_and_cache it feeds (attention_backend.py:86-88). */
int kvq_int8_quant_scatter(const void* key, const void* value, int dtype,
                           const void* k_inv, const void* v_inv,
                           const void* slot_mapping, int slot_index_type, int64_t num_tokens,
                           int64_t channels, int8_t* key_cache, int8_t* value_cache,
                           int64_t num_blocks, int block_size, void* stream);

/* Paged int8 -> dense TND in the activation dtype: (x - 0) * aq, rounded to
 * `dtype`.  Rows of request b are [cu_seqlens[b], cu_seqlens[b+1]).
 * Replaces _dequant_int8_paged_kv_to_dense (attention_backend.py:370-404). */
int kvq_int8_dequant_gather(const int8_t* key_cache, const int8_t* value_cache,
                            int64_t num_blocks, int block_size, int num_kv_heads, int head_size,
                            const void* k_aq, const void* v_aq, int dtype,
                            const int32_t* block_table, int64_t max_blocks,
                            const int64_t* cu_seqlens, int64_t batch,
                            void* out_k, void* out_v, void* stream);

/* Fused INT8 decode attention with per-channel antiquant (offset 0):
 * K = int8 * k_aq[h, d], V = int8 * v_aq[h, d].
 *   query/out [batch, num_heads, D] of `dtype`; k_aq/v_aq [KVH*D] of `dtype`
 *   seq_meta int32 [batch, 4] = {seq_len, first_work, num_work, unused}
 *   work     int32 [num_work, 4] = {request, pos_begin, pos_end, kind}
 * Replaces _forward_int8_decode (attention_backend.py:173-205):
 * npu_fused_infer_attention_score BNSD with key/value_antiquant_scale. */
int64_t kvq_int8_decode_workspace_bytes(int64_t num_work, int num_heads, int head_size);
int kvq_int8_decode_attn(const void* query, int dtype, int64_t batch, int num_heads,
                         int num_kv_heads, int head_size, float scale,
                         const int8_t* key_cache, const int8_t* value_cache,
                         int64_t num_blocks, int block_size,
                         const void* k_aq, const void* v_aq,
                         const int32_t* block_table, int64_t max_blocks,
                         const int32_t* seq_meta, const int32_t* work, int64_t num_work,
                         void* workspace, void* out, void* stream);

/* ---- fp8_per_token_head ------------------------------------------------- */

/* Quantize [num_tokens, KVH, D] K/V (D % 4 == 0, D <= 512; D <= 256 when
 * D % 8 != 0) to OCP E4M3 codes with one fp32 scale per (token, head) and
 * write them by slot into k_data/v_data [NB, Bs, KVH, D] bytes and
 * k_scale/v_scale [NB, Bs, KVH] fp32:
 *   scale = max(amax|x| / 448, 1e-6), code = e4m3fn(clamp(x / scale, +-448))
 * with IEEE division and round to nearest even.  Negative slots (padding)
 * and slots >= NB*Bs are skipped.
 * Replaces the host store kernel _per_token_head_store_kernel and its wrapper
 * fp8_per_token_head_store (pkg/ops/triton/per_token_head_store.py:141-294),
 * with the arithmetic of Fp8PerTokenHeadSemantics.quantize
 * (pkg/methods/fp8_per_token_head/semantics.py:52-61). */
int kvq_fp8_pth_store(const void* key, const void* value, int dtype,
                      const void* slot_mapping, int slot_index_type, int64_t num_tokens,
                      int num_kv_heads, int head_size, uint8_t* k_data, float* k_scale,
                      uint8_t* v_data, float* v_scale, int64_t num_blocks, int block_size,
                      void* stream);

/* Paged E4M3 -> dense TND [cu_seqlens[batch], KVH, D] of out_dtype:
 * x = float(code) * scale in fp32, then rounded to out_dtype.  Rows of request
 * b are [cu_seqlens[b], cu_seqlens[b+1]); block ids < 0 read page 0 and ids
 * >= num_blocks read the last page (callers check live ids on the host).
 * The read path of Fp8PerTokenHeadSemantics.dequantize
 * (pkg/methods/fp8_per_token_head/semantics.py:63-65) over the byte layout of
 * pkg/methods/fp8_per_token_head/byte_cache.py:13-27; the reference has no
 * device read path for this scheme. */
int kvq_fp8_pth_gather(const uint8_t* k_data, const float* k_scale, const uint8_t* v_data,
                       const float* v_scale, int64_t num_blocks, int block_size,
                       int num_kv_heads, int head_size, const void* block_table,
                       int block_index_type, int64_t max_blocks, const int64_t* cu_seqlens,
                       int64_t batch, void* out_k, void* out_v, int out_dtype, void* stream);

/* ---- self-test ---------------------------------------------------------- */

/* One v_mfma_f32_16x16x32_f16 with the operand/result lane mapping the decode
 * kernels assume: d[16x16] = a[16x32] * b[32x16], row-major fp16 inputs and
 * fp32 output.  No counterpart in the reference; it lets the test suite pin
 * the gfx950 matrix-core lane layout directly. */
int kvq_selftest_mfma_f16(const void* a, const void* b, float* d, void* stream);

/* One wave copies src[0..320) uint32 through LDS with the LDS-DMA loads the
 * decode kernel stages its tiles with (global_load_lds, 16-byte lanes for
 * words 0..255, 4-byte lanes for words 256..319) and writes the LDS image to
 * dst[0..320); dst == src pins the lane -> LDS address mapping.  No
 * counterpart in the reference. */
int kvq_selftest_lds_dma(const void* src, void* dst, void* stream);

/* One wave applies the cross-lane reductions the kernels use to 16 rounds of
 * 64 floats src[64 t + l] and writes, for lane l of round t,
 * dst[6 (64 t + l) + 0..5] = the max over lanes l, l^16, l^32, l^48
 * (permlane row swaps), their sum as (x_l + x_l^16) + (x_l^32 + x_l^48), the
 * max and the sum over all 64 lanes (DPP steps plus the row swaps), and the
 * four-row maxima of round t and of round (t + 1) % 16 taken together (the
 * paired form).  No counterpart in the reference; it pins the gfx950 lane
 * semantics. */
int kvq_selftest_lane_reductions(const float* src, float* dst, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KVQ_HIP_H_ */
