/*
 * nanokv.h -- C ABI of the MI355X-native NanoKV sparse-attention layer-step.
 *
 * One shared library (libnanokv.so, gfx950 code objects) exports the entry
 * points below.  Every pointer is a device pointer unless the comment says
 * otherwise; every entry point enqueues work on `stream` (a hipStream_t) and
 * returns without synchronising.  The caller owns every buffer, including
 * workspaces; nothing here allocates device memory.  Return value: NKV_OK, or
 * an NKV_ERR_* code with a message available from nkv_last_error().
 *
 * Store layout (one allocation per field, leading layer dimension L):
 *   hist_k / hist_v : [L][Hkv][cap][B][D]  bf16 (NKV_KV_BF16) or int8
 *   reps            : [L][Hkv][cap][r][D]  bf16
 *   sink_k / sink_v : [L][Hkv][S][D]       bf16
 *   recent_k/_v     : [L][Hkv][R][D]       bf16 ring; logical slot i of the
 *                      reference's left-aligned recent buffer lives at
 *                      physical slot (ring_start + i) % R
 *   k_scale         : [L][Hkv][D] fp32     (NKV_KV_INT8_CHANNEL)
 *   v_scale         : [L][Hkv][cap] fp32   (NKV_KV_INT8_CHANNEL)
 *   k_tscale/v_tscale: [L][Hkv][cap*B] fp16 (NKV_KV_INT8_TOKEN)
 * B = 64 and D = 128 are fixed by the kernels; Hq/Hkv <= 16; r in {1,2,4,8}.
 *
 * Reference citations are to Tao20060602/nano-vllm-kv-optimizer.
 */
#ifndef NANOKV_H
#define NANOKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NKV_ABI_VERSION 1

enum nkv_status {
  NKV_OK = 0,
  NKV_ERR_ARG = 1,          /* an argument violates a documented constraint */
  NKV_ERR_UNSUPPORTED = 2,  /* shape/format outside what the kernels handle */
  NKV_ERR_HIP = 3           /* a HIP launch or runtime call failed */
};

enum nkv_kv_format {
  NKV_KV_BF16 = 0,
  NKV_KV_INT8_CHANNEL = 1,  /* K per-(Hkv,D) scale, V per-(block,Hkv) scale: m12_runtime.py:460-477 */
  NKV_KV_INT8_TOKEN = 2     /* per-token-per-KV-head fp16 scales for K and V */
};

enum nkv_topk_order {
  NKV_ORDER_SCORE_DESC = 0, /* torch.topk(sorted=True); ties by block id ascending */
  NKV_ORDER_ID_ASC = 1      /* the same set, ids ascending (gather_sort) */
};

/* Plain-data view of a model's HBM-resident sparse KV store. */
typedef struct nkv_store {
  void* hist_k;
  void* hist_v;
  void* reps;
  void* sink_k;
  void* sink_v;
  void* recent_k;
  void* recent_v;
  float* k_scale;
  float* v_scale;
  uint16_t* k_tscale;
  uint16_t* v_tscale;
  int32_t num_layers;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t block_size;
  int32_t r;
  int32_t cap_blocks;
  int32_t sink_tokens;
  int32_t recent_tokens;
  int32_t kv_format;
} nkv_store;

int nkv_abi_version(void);
/* Thread-local message of the last failing call on this host thread (host memory). */
const char* nkv_last_error(void);

/*
 * Block scoring + Top-K selection for `num_layers` layers starting at
 * `layer0`.
 *
 * Replaces M12LayerRuntime._gpu_select fixed-budget path
 * (nanovllm/sparse/m12_runtime.py:959-1055; scorer fused_select.py:23-79) and,
 * with per_query=1, the per-query Top-K of _gpu_select_per_query
 * (m12_runtime.py:1057-1079).
 *
 * q        : bf16 [num_layers][nq][Hq][D], layer stride q_layer_stride elements.
 * score[b] = max over (n<nq, h, g, j<r) of the fp32 dot q[n][h*G+g] . reps[h][b][j],
 *            each dot accumulated in ascending d with fma from +0
 *            (per_query=0); per n when per_query=1.  A NaN dot makes the
 *            score NaN, which ranks above +inf; -0 ranks as +0.
 * Protected ids (device int32 list, shared by all layers; ids outside
 * [0, nblocks) are ignored) are scored -inf.  k_eff = min(k, max(1, nblocks
 * - |protected in range|)) ids are returned per (layer[, n]), ordered by
 * `order`; exact ties go to the lower block id.
 * score_keys : uint32 workspace [num_layers][nq'][nblocks] (nq' = per_query ?
 *              nq : 1) that must be zero before the first call; every call
 *              leaves it zero.  Calls that share one workspace must not overlap.
 * out_scores : fp32 [num_layers][nq'][nblocks] raw scores (before the
 *              protected mask), or NULL.
 * out_ids    : int32 [num_layers][nq'][k] (entries >= k_eff untouched).
 * out_vals   : fp32  [num_layers][nq'][k] selected scores, or NULL.
 * Constraints: 1 <= nblocks <= cap_blocks, nblocks <= 12288, 1 <= k <= 1024,
 *              nq <= 64.
 */
int nkv_select(const nkv_store* st, int layer0, int num_layers,
               const uint16_t* q, int64_t q_layer_stride, int nq, int per_query,
               int nblocks, const int32_t* protected_ids, int n_protected,
               int k, int order, uint32_t* score_keys, float* out_scores,
               int32_t* out_ids, float* out_vals, void* stream);

/*
 * Segmented GQA attention for few queries (decode and speculative verify).
 *
 * Replaces, for decode, M12LayerRuntime.decode steps 1 and 3-5
 * (m12_runtime.py:1164-1172 recent shift/append, :1212-1311 gather + pack,
 * :1317-1320 -> _fused_attention fast path :867-873); for verify,
 * verify_tokens steps 2-3 (m12_runtime.py:686-758) with the masked
 * _fused_attention path (:875-896) and the lossless per-query mask (:753-758).
 *
 * Keys/values attended by query t of layer l, KV head h (as one softmax):
 *   n_hist selected history blocks ids[l][i] (64 tokens each; with
 *            `allowed` != NULL only blocks with allowed[t][i] != 0),
 *   sink   : sink[l][h][0 .. sink_len),
 *   recent : ring slots whose logical position (slot - ring_base) mod R lies
 *            in [rec_lo, rec_lo + rec_len),
 *   chunk  : new tokens k_new/v_new[l][c], c < n_chunk, causal (query t sees
 *            c <= t).  Decode passes its new token as a one-token chunk.
 * If write_slot >= 0 the call also stores chunk token 0 into ring slot
 * write_slot (decode's shift + append); that slot must lie outside the
 * attended recent window.
 * q      : bf16 [num_layers][tq][Hq][D] (layer stride q_layer_stride).
 * k_new, v_new : bf16 [num_layers][n_chunk][Hkv][D] (layer stride kv_layer_stride).
 * ids    : int32 [num_layers][ids_layer_stride]; ids outside [0, cap) attend
 *          nothing (and cost no loads: a union padded with -1 is fine).
 * allowed: uint8 [tq][n_hist] per layer, layer stride allowed_layer_stride
 *          (0: one mask shared by all layers, else >= tq * n_hist), or NULL.
 * out    : bf16 [num_layers][tq][Hq][D] (layer stride q_layer_stride).
 * partial_ws : fp32 workspace, >= nkv_attend_workspace_floats(...) floats
 *              (unused when splits == 1).
 * splits : workgroups per (layer, KV head, query group), 1..64; with
 *          splits > 1 a second kernel on the same stream merges the partial
 *          softmax states.  Queries are processed in groups of 16/G per
 *          workgroup (grid z = layers x groups).  splits = 0 (groups of at
 *          most 4 query rows, tq * G <= 4, e.g. one decode token at G = 4):
 *          the stream form -- one resident round of wavefronts (two
 *          workgroups per CU, at most 2048 wavefronts), the same number per
 *          (layer, KV head, group), each taking an equal run of its group's
 *          segments and writing one partial, and the merge kernel combines
 *          them.  splits = 0 with 17-32 query rows per group
 *          (the wide few-query kernel, e.g. verify's 6 draft tokens at
 *          G = 4): a tiered plan -- the first groups in larger pieces
 *          filling one round of workgroups, the rest in pieces about 3/4
 *          that size filling a second (one workgroup per group once the
 *          groups alone fill the device).  Other shapes return
 *          NKV_ERR_UNSUPPORTED.
 * Constraints: 1 <= tq <= 65536, n_hist <= 4096, n_chunk in {0, tq};
 *          fp32 softmax and accumulation.
 */
int nkv_attend(const nkv_store* st, int layer0, int num_layers,
               const uint16_t* q, int64_t q_layer_stride, int tq,
               const uint16_t* k_new, const uint16_t* v_new, int64_t kv_layer_stride,
               int n_chunk, int write_slot,
               const int32_t* ids, int64_t ids_layer_stride, int n_hist,
               const uint8_t* allowed, int64_t allowed_layer_stride, int sink_len,
               int ring_base, int rec_lo, int rec_len,
               float scale, int splits,
               float* partial_ws, uint16_t* out, void* stream);

/* Floats of partial_ws needed by nkv_attend for these sizes. */
int64_t nkv_attend_workspace_floats(int num_layers, int num_kv_heads, int num_heads,
                                    int tq, int splits);

/*
 * Timing marks around the attention kernel.  No counterpart in the
 * reference (its attention is one library call); for callers that time the
 * attention kernel apart from the selection before it and the split merge
 * after it with events of their own.  While set, every launch of the
 * few-query attention kernels made by this host thread -- nkv_attend,
 * nkv_decode_step*, and nkv_attend_packed below its matrix-core threshold --
 * records `before` (a hipEvent_t) on the launch stream right before the
 * attention kernel and `after` right after it, ahead of the split merge if
 * there is one.  NULL (the initial state of both) turns a mark off.  Per
 * host thread; the library never creates or destroys the events.
 */
int nkv_set_attend_marks(void* before, void* after);

/*
 * The whole sparse decode layer-step for `num_layers` layers in one call:
 * nkv_select (per_query=0, NKV_ORDER_SCORE_DESC, no out_scores / out_vals)
 * then nkv_attend (tq = 1, n_chunk = 1, allowed = NULL) for every layer.
 *
 * Replaces steps 2 + 5 (with the recent-ring append of step 1) of
 * M12LayerRuntime.decode (nanovllm/sparse/m12_runtime.py:1141-1346) for a
 * batch of independent layers.
 *
 * The layers are split into min(nstreams, num_layers) contiguous ranges;
 * range r is enqueued on streams[r] (streams[0] is the caller's stream; the
 * others first wait for the work already on streams[0], and streams[0] waits
 * for all of them before this returns).  Each range makes exactly the
 * launches a single-range call would for its layers, so results do not
 * depend on nstreams.  The first multi-stream call on a host thread creates
 * nstreams events (no timing, no system-scope fence) for the current
 * device, kept for the thread's lifetime.
 * q, out : bf16 [num_layers][1][Hq][D]; k_new, v_new: bf16 [num_layers][1][Hkv][D]
 *          (contiguous).
 * score_keys : as nkv_select, [num_layers][nblocks].
 * out_ids    : int32 [num_layers][k]; n_hist: the ids attended per layer
 *              (k_eff of nkv_select, 1 <= n_hist <= k).
 * sink_len, write_slot, ring_base, rec_lo, rec_len, scale, splits: as nkv_attend
 *          (splits 0: the stream form).
 * partial_ws : >= nkv_decode_step_workspace_floats(...) floats (splits != 1).
 */
int nkv_decode_step(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                    const uint16_t* k_new, const uint16_t* v_new, int nblocks,
                    const int32_t* protected_ids, int n_protected, int k, int n_hist,
                    int sink_len, int write_slot, int ring_base, int rec_lo, int rec_len,
                    float scale, int splits, uint32_t* score_keys, int32_t* out_ids,
                    float* partial_ws, uint16_t* out, int nstreams, void* const* streams);

/* Floats of partial_ws needed by nkv_decode_step (one attention workspace per range). */
int64_t nkv_decode_step_workspace_floats(int num_layers, int num_kv_heads, int num_heads,
                                         int splits, int nstreams);

/*
 * nkv_decode_step without caller workspaces and without any allocation.
 * No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 *
 * Same arguments and results as nkv_decode_step with one range on `stream`,
 * except that score_keys and partial_ws live in a 16 MiB array in the
 * library's device code object, one per GPU, held until the process ends:
 * 1 MiB of score keys (num_layers x nblocks <= 262144) and 15 MiB of split
 * partials (nkv_attend_workspace_floats(num_layers, Hkv, Hq, 1, splits) <=
 * 3932160 floats: 16 x 130 per layer, KV head and split, e.g. 36 layers x 8
 * KV heads x up to 6 splits; the stream form, splits 0, needs
 * (2048 + num_layers x Hkv) x 4 x 130).  Larger sizes
 * are rejected with NKV_ERR_ARG before any device work.  The first call on a
 * device looks the array up (hipGetSymbolAddress) and clears its key region
 * with a fill kernel on `stream`; every call leaves the keys it used at zero.
 * All calls on one GPU share the array: calls that overlap (other streams,
 * other host threads) race and must be serialised by the caller.
 */
int nkv_decode_step_noalloc(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                            const uint16_t* k_new, const uint16_t* v_new, int nblocks,
                            const int32_t* protected_ids, int n_protected, int k, int n_hist,
                            int sink_len, int write_slot, int ring_base, int rec_lo, int rec_len,
                            float scale, int splits, int32_t* out_ids, uint16_t* out, void* stream);

/*
 * The steady-state decode layer-step (recent window full) with the ring
 * position in device memory, so that every argument is the same from one
 * step to the next and the call can be captured in a HIP graph and replayed.
 *
 * Same work as nkv_decode_step with one range (nkv_select, then nkv_attend
 * over [selected | sink | the R - 1 recent tokens | the new token]), for
 * M12LayerRuntime.decode (nanovllm/sparse/m12_runtime.py:1141-1346) once
 * valid_len >= R - 1.
 * ring_start : int32 [num_layers] device array: each layer's ring start, the
 *              physical slot of its oldest recent token, which this step's
 *              new token overwrites (the attended ring part starts one slot
 *              after it).  Values are taken mod R.  After the attention the
 *              split merge (with splits = 1, a one-workgroup kernel) advances
 *              each entry by one slot (mod R).
 * score_keys : as nkv_select, [num_layers][nblocks].
 * partial_ws : >= nkv_attend_workspace_floats(num_layers, Hkv, Hq, 1, splits)
 *              floats (splits != 1; splits 0: the stream form).
 * Other arguments as nkv_decode_step.
 */
int nkv_decode_step_ring(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                         const uint16_t* k_new, const uint16_t* v_new, int nblocks,
                         const int32_t* protected_ids, int n_protected, int k, int n_hist,
                         int sink_len, int32_t* ring_start, float scale, int splits,
                         uint32_t* score_keys, int32_t* out_ids, float* partial_ws, uint16_t* out,
                         void* stream);

/*
 * Union of per-query selections, for lossless speculative verify.
 *
 * Replaces the host-side union + mask of M12LayerRuntime._gpu_select_per_query
 * (nanovllm/sparse/m12_runtime.py:1057-1087: torch.unique of the per-query
 * Top-K ids, searchsorted, scatter into `allowed`) for num_layers layers at
 * once, on the device, so verify needs no device-to-host round trip.
 *
 * ids         : int32 [num_layers][tq][k], the per-query selections of
 *               nkv_select (per_query = 1); the first k_eff of each row are used.
 * out_union   : int32 [num_layers][umax]: the distinct ids ascending, then -1.
 * out_count   : int32 [num_layers]: the union sizes.
 * out_allowed : uint8 [num_layers][tq][umax]: 1 where union[u] is among
 *               query t's ids (0 past the union).
 * Feed out_union (n_hist = umax) and out_allowed (allowed_layer_stride =
 * tq * umax) to nkv_attend / nkv_prefill_attend.
 * Constraints: 1 <= tq <= 16, 1 <= k_eff <= k, tq * k_eff <= 4096,
 *              umax >= tq * k_eff; ids in [0, 12288) (the block ids
 *              nkv_select returns; other values are left out of both outputs).
 */
int nkv_select_union(const int32_t* ids, int num_layers, int tq, int k, int k_eff, int umax,
                     int32_t* out_union, int32_t* out_count, uint8_t* out_allowed, void* stream);

/*
 * Per-query selection and its union in two launches: the scorer of
 * nkv_select (per_query = 1), then one workgroup per layer that takes each
 * query's Top-K (the selection, order NKV_ORDER_SCORE_DESC, of nkv_select)
 * and forms the union and mask of those ids (nkv_select_union) without a
 * launch in between.
 *
 * Replaces M12LayerRuntime._gpu_select_per_query whole
 * (nanovllm/sparse/m12_runtime.py:1057-1087: scores per query, torch.topk per
 * query, torch.unique, searchsorted, scatter into `allowed`).
 *
 * Outputs: those of nkv_select (score_keys left zeroed, out_scores, out_ids
 * [num_layers][nq][k], out_vals) and of nkv_select_union with tq = nq and
 * k_eff = the number of ids each row holds (min(k, selectable blocks)).
 * Constraints: 1 <= nq <= 16, 1 <= k <= 64, 1 <= nblocks <= 2048,
 *              umax >= nq * min(k, nblocks); others as nkv_select.
 */
int nkv_select_per_query(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                         int64_t q_layer_stride, int nq, int nblocks, const int32_t* protected_ids,
                         int n_protected, int k, uint32_t* score_keys, float* out_scores, int32_t* out_ids,
                         float* out_vals, int umax, int32_t* out_union, int32_t* out_count,
                         uint8_t* out_allowed, void* stream);

/*
 * Segmented causal GQA attention for a chunk of many queries, on the matrix
 * cores (bf16 MFMA for Q.K^T and P.V, fp32 softmax and accumulation).
 *
 * Replaces the attention of M12LayerRuntime.prefill_chunk: the pack of
 * [selected | sink | previous recent | chunk] (m12_runtime.py:560-636) and
 * _prefill_attention's bottom-right causal flash attention over it
 * (:809-839; same function as the masked _fused_attention path :875-896).
 * int8 history blocks are dequantised to bf16(code * scale) as the
 * reference's pack does (m12_runtime.py:1262-1267, fused_dequant.py:34-44).
 *
 * Same key set and argument meaning as nkv_attend with n_chunk = tq (query t
 * is chunk token t and sees chunk tokens c <= t) and write_slot = -1.
 * Queries are tiled 128/G tokens x G heads per workgroup (G = Hq / Hkv must
 * divide 128).  splits > 1 cuts each tile's segment list into that many
 * workgroups (few tiles: short chunks, verify) whose partial softmax states a
 * second kernel on the same stream merges; partial_ws then needs
 * nkv_prefill_workspace_floats(...) floats.
 * Constraints: 1 <= tq <= 65536, n_hist <= 4096, 1 <= splits <= 64.
 */
int nkv_prefill_attend(const nkv_store* st, int layer0, int num_layers,
                       const uint16_t* q, int64_t q_layer_stride, int tq,
                       const uint16_t* k_new, const uint16_t* v_new, int64_t kv_layer_stride,
                       const int32_t* ids, int64_t ids_layer_stride, int n_hist,
                       const uint8_t* allowed, int64_t allowed_layer_stride, int sink_len,
                       int ring_base, int rec_lo, int rec_len,
                       float scale, int splits, float* partial_ws, uint16_t* out, void* stream);

/* Floats of partial_ws needed by nkv_prefill_attend (0 when splits == 1). */
int64_t nkv_prefill_workspace_floats(int num_layers, int num_kv_heads, int num_heads, int tq,
                                     int splits);

/*
 * nkv_prefill_attend with one history selection per tile of `sel_tile`
 * queries instead of one per chunk: query t attends the n_hist blocks
 * ids[l][(t / sel_tile) * ids_tile_stride + i], then the sink, the previous
 * recent window and the chunk (causal), as nkv_prefill_attend.  No reference
 * counterpart: the reference selects once per chunk from its query summaries
 * (m12_runtime.py:550-556); this is that selection applied to each tile of a
 * chunk (the per-tile summaries come from nkv_query_summaries, the per-tile
 * ids from nkv_select with per_query = 1).  No per-query mask.
 * Constraints: sel_tile a positive multiple of 128 / G tokens (the
 * workgroup's query tile); ids_tile_stride >= n_hist; ids_layer_stride >=
 * ceil(tq / sel_tile) * ids_tile_stride; otherwise as nkv_prefill_attend
 * (partial_ws: nkv_prefill_workspace_floats floats when splits > 1).
 */
int nkv_prefill_attend_tiled(const nkv_store* st, int layer0, int num_layers,
                             const uint16_t* q, int64_t q_layer_stride, int tq,
                             const uint16_t* k_new, const uint16_t* v_new, int64_t kv_layer_stride,
                             const int32_t* ids, int64_t ids_layer_stride, int64_t ids_tile_stride,
                             int sel_tile, int n_hist, int sink_len, int ring_base, int rec_lo,
                             int rec_len, float scale, int splits, float* partial_ws, uint16_t* out,
                             void* stream);

/*
 * Exact attention over caller-packed keys: M12LayerRuntime._fused_attention
 * (nanovllm/sparse/m12_runtime.py:845-896), the reference's inspectable
 * attention over [selected | sink | recent | chunk] that its packing paths
 * and tests call.
 *
 * q    : bf16 [tq][num_heads][D];  k, v : bf16 [s_len][num_kv_heads][D]
 *        (token-major, as the reference packs them).
 * Query t, head hq (KV head hq / G) sees key j iff j - causal_from <= t and
 * (mask == NULL or mask[t][j] == 0): the reference's mask
 * (cols >= t + causal_from + 1) & (cols >= causal_from), OR'd with its
 * attn_mask (True = disallowed).  causal_from >= s_len = every key visible
 * (the decode fast path).
 * mask : uint8 [tq][s_len], nonzero = hidden, or NULL.
 * out  : bf16 [tq][num_heads][D].
 * Queries of more than 16 / G tokens run on the matrix-core kernel (P enters
 * P.V rounded to bf16, as flash-attention's; the reference's torch backend is
 * fp32), fewer on the few-query kernel (fp32-accurate P.V).  splits: as
 * nkv_attend / nkv_prefill_attend; partial_ws >=
 * nkv_attend_packed_workspace_floats(...) floats when splits > 1.
 * Constraints: G = num_heads / num_kv_heads in {1, 2, 4, 8, 16}, D = 128,
 *              1 <= tq <= 65536, 1 <= s_len <= 2^20.
 */
int nkv_attend_packed(int num_heads, int num_kv_heads, const uint16_t* q, int tq,
                      const uint16_t* k, const uint16_t* v, int s_len, int causal_from,
                      const uint8_t* mask, float scale, int splits, float* partial_ws,
                      uint16_t* out, void* stream);

/* Floats of partial_ws needed by nkv_attend_packed (0 when splits == 1). */
int64_t nkv_attend_packed_workspace_floats(int num_heads, int num_kv_heads, int tq, int splits);

/*
 * Append one prefill chunk to the history of `num_layers` layers.
 *
 * Replaces the history / quantisation / sink part of M12LayerRuntime._store_kv
 * (m12_runtime.py:420-481; quant_kv.py:27-49): tokens k[t], v[t] (bf16
 * [num_layers][T][Hkv][D], layer stride kv_layer_stride) go to blocks
 * start_block .. start_block + ceil(T/64) - 1, the last one zero-padded.
 * int8 channel format: if compute_k_scale, k_scale[l] is first set from this
 * chunk (amax/127, clamped at 1e-8/127); V gets a per-block scale.
 * int8 token format: per-token fp16 scales.
 * If write_sink, sink[l][h][0 .. min(S, T)) = the chunk's first tokens.
 * Constraints: T >= 1, start_block + ceil(T/64) <= cap_blocks.
 */
int nkv_store_chunk(const nkv_store* st, int layer0, int num_layers,
                    const uint16_t* k, const uint16_t* v, int64_t kv_layer_stride,
                    int T, int start_block, int compute_k_scale, int write_sink,
                    void* stream);

/*
 * Block representatives of the chunk's blocks.
 *
 * Replaces M12LayerRuntime._build_reps_gpu (m12_runtime.py:354-395): per
 * (block, KV head) the first argmax of cos(k_t, mean direction), then r-1
 * farthest-point steps (first argmin of the max cos to the chosen set); the
 * chosen raw bf16 keys go to reps[l][h][start_block + b][j].
 * k: bf16 [num_layers][T][Hkv][D] (tokens >= T of the last block are zeros).
 */
int nkv_build_reps(const nkv_store* st, int layer0, int num_layers,
                   const uint16_t* k, int64_t kv_layer_stride, int T,
                   int start_block, void* stream);

/*
 * Recent-window update on the logical buffer.
 *
 * Replaces the recent part of _store_kv (m12_runtime.py:486-503) and of
 * commit_verified (m12_runtime.py:784-800): logical slots [0, carry) take the
 * old logical slots [old_len - carry, old_len), then slots
 * [carry, carry + n_src) take src tokens src_lo .. src_lo + n_src - 1 of k/v
 * (bf16 [num_layers][*][Hkv][D]).  Slots >= carry + n_src keep their content.
 */
int nkv_recent_update(const nkv_store* st, int layer0, int num_layers,
                      const uint16_t* k, const uint16_t* v, int64_t kv_layer_stride,
                      int src_lo, int n_src, int ring_start, int old_len, int carry,
                      void* stream);

/*
 * Query summaries for prefill routing.
 *
 * Replaces prefill_query_summaries (m12_runtime.py:53-67): out[l][s] =
 * bf16 round-to-nearest-even of the mean of q[l][lo_s .. hi_s) (torch
 * tensor_split bounds over T tokens, nseg = min(nsegments, T)).
 * q: bf16 [num_layers][T][Hq][D]; out: bf16 [num_layers][nseg][Hq][D].
 */
int nkv_query_summaries(const uint16_t* q, int64_t q_layer_stride, int num_layers,
                        int T, int num_heads, int head_dim, int nsegments,
                        uint16_t* out, int64_t out_layer_stride, void* stream);

/*
 * Device address of pinned host memory, for a history kept in host memory.
 *
 * Replaces the reference's host-resident history and its per-step gather +
 * H2D copy of the selected blocks into pinned staging (m12_runtime.py:185-246
 * allocation, :1212-1311 decode gather, :560-636 prefill gather): a store
 * whose hist_k / hist_v point at pinned host memory (allocated by the HIP
 * runtime: hipHostMalloc, or torch's pin_memory=True) is read in place by
 * every kernel over the host link, so no staging copy exists.  Put the
 * returned address (not host_ptr) in nkv_store.hist_k / hist_v.
 * Returns NKV_ERR_ARG when host_ptr is not pinned host memory of the HIP
 * runtime or is not mapped for the current device.
 */
int nkv_host_device_pointer(const void* host_ptr, void** device_ptr);

/* ------------------------------------------------------------------------
 * Fused elementwise ops of the Qwen3 decoder that calls the layer-step
 * (nanovllm/models/qwen3.py).  bf16 tensors, contiguous rows, device
 * pointers; each call is one launch on `stream`.
 * ---------------------------------------------------------------------- */

/*
 * RMSNorm of `rows` rows of n elements, optionally after a residual add
 * (RMSNorm.forward, nanovllm/layers/layernorm.py:17-44):
 *   s = x (+ residual) in fp32; residual_out = bf16(s) (if non-NULL);
 *   out = bf16(bf16(s * rsqrt(mean(s^2) + eps)) * weight).
 * n: a multiple of 8, at most 8192; buffers 16-byte aligned.
 */
int nkv_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, uint16_t* out,
                uint16_t* residual_out, int rows, int n, float eps, void* stream);

/*
 * Qwen3Attention's q/k RMSNorm and RoPE (nanovllm/models/qwen3.py:99-110,
 * nanovllm/layers/rotary_embedding.py:6-50) on the fused projection output
 * qkv [rows][Hq + 2 Hkv][128]: per head of q and k, RMSNorm over the 128 dims
 * with q_weight / k_weight, then rotate-half RoPE in fp32 with
 * cos/sin_table [max_position][64] at positions[row] (int64; clamped to
 * [0, max_position)); v is copied.  Outputs q [rows][Hq][128], k and v
 * [rows][Hkv][128].
 */
int nkv_qk_norm_rope(const uint16_t* qkv, int rows, int num_heads, int num_kv_heads, const uint16_t* q_weight,
                     const uint16_t* k_weight, const float* cos_table, const float* sin_table, int max_position,
                     const int64_t* positions, float eps, uint16_t* q, uint16_t* k, uint16_t* v, void* stream);

/*
 * SiLU-and-mul (nanovllm/layers/activation.py:6-11) of gate_up
 * [rows][2 intermediate] (gate, then up) -> out [rows][intermediate]:
 * out = bf16(bf16(g / (1 + e^-g)) * u).  intermediate: a multiple of 8;
 * buffers 16-byte aligned.
 */
int nkv_silu_mul(const uint16_t* gate_up, uint16_t* out, int rows, int intermediate, void* stream);

/*
 * y [m][n] = x [m][k] . weight [n][k]^T (nn.Linear without bias, the decode-
 * time projections of nanovllm/layers/linear.py) for 1 <= m <= 4 rows:
 * fp32 accumulation, bf16 output.  k: a multiple of 8; weight and x 16-byte
 * aligned.
 */
int nkv_gemv(const uint16_t* weight, const uint16_t* x, uint16_t* y, int m, int n, int k, void* stream);

/*
 * Qwen3MLP's gate|up projection and SiLU-and-mul in one launch for 1 <= m <= 4
 * rows (nanovllm/models/qwen3.py:125-130, nanovllm/layers/activation.py:6-11):
 * gate_up_weight [2 intermediate][k] (gate rows, then up rows), x [m][k] ->
 * y [m][intermediate] = bf16(bf16(silu(g)) * u) with g, u the bf16-rounded
 * products, the rounding points of nkv_gemv followed by nkv_silu_mul.
 */
int nkv_gemv_silu_mul(const uint16_t* gate_up_weight, const uint16_t* x, uint16_t* y, int m, int intermediate,
                      int k, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOKV_H */
