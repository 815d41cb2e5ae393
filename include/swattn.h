/*
 * swattn.h -- C ABI of libswattn.so, the MI355X (gfx950) Switch Attention
 * prefill library.
 *
 * Every entry point takes device pointers, plain sizes and a hipStream_t
 * (passed as void*; NULL = the legacy default stream), enqueues its kernels on
 * that stream and returns without synchronising.  Nothing here allocates
 * device memory: scratch space is passed in by the caller.  bf16 row tensors
 * (q, k, v, out and their gradients, KV caches, merge partials) must be
 * 16-byte aligned, and workspaces 256-byte aligned (as hipMalloc returns);
 * a misaligned one is rejected with SWATTN_EINVAL.
 *
 * Return value: SWATTN_OK (0) on success, a negative SWATTN_E* code for an
 * invalid argument detected on the host, or a positive hipError_t from the
 * launch.  swattn_last_error() gives a message for the calling thread.
 *
 * Reference tags: V = swiattn_gqa_prefill_varlen.py,
 *                 F = swiattn_gqa_prefill.py  (YushengZhao/SwitchAttentionKernels)
 */
#ifndef SWATTN_H_
#define SWATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SWATTN_OK 0
#define SWATTN_EINVAL (-1)      /* bad size, null pointer or unsupported shape */
#define SWATTN_EWORKSPACE (-2)  /* workspace smaller than required            */

/* Error bits written by swattn_check_indices, in the order the reference
 * raises them (V:384-393). */
#define SWATTN_ERR_FULL_RANGE 1   /* V:299-300 "query index is outside [0, sequence_length)" */
#define SWATTN_ERR_FULL_ORDER 2   /* V:301-302 "query indices must be strictly increasing"   */
#define SWATTN_ERR_LOCAL_RANGE 4  /* V:299-300, local list                                    */
#define SWATTN_ERR_LOCAL_ORDER 8  /* V:301-302, local list                                    */
#define SWATTN_ERR_OVERLAP 16     /* a position in both lists (contract of V:341-342)         */

/* Library version, (major << 16) | minor.  0.2 changed the signature of
 * swattn_prefill_bwd_workspace_bytes (a window argument before n_full) and
 * took the MFMA-rate probe out of this library; callers built against 0.1
 * must be rebuilt. */
int swattn_version(void);

/* Message for the last non-zero status returned on the calling thread. */
const char* swattn_last_error(void);

/*
 * Router-mask compaction.  Replaces build_switch_query_indices (V:306-322),
 * whose body is `arange(S)[mask], arange(S)[~mask]` over torch's nonzero.
 *
 *   mask     n bytes, nonzero = routed to full causal attention.  A [B, S]
 *            mask is passed flattened; positions are then b*S + i.
 *   indices  n int32 outputs: the ascending full list in [0, nf), followed by
 *            the ascending local list in [nf, n).
 *   counts   2 int32 outputs: {nf, n - nf}.
 *   workspace/workspace_bytes: at least swattn_compact_workspace_bytes(n).
 * Bit-exact with the reference: both lists are the stable compaction.
 */
size_t swattn_compact_workspace_bytes(int64_t n);
int swattn_compact(const uint8_t* mask, int64_t n, int32_t* indices, int32_t* counts,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * Router logits -> the same two lists as swattn_compact, in one pass.
 * No counterpart in the reference, whose router is outside its kernels
 * (README:85, V:4-5, V:309-310): this fuses the `logits > threshold` mask
 * a caller builds before build_switch_query_indices (V:306-322), so that
 * neither the mask nor its extra pass over HBM exists.
 *
 *   logits     n values of type dtype (SWATTN_DTYPE_*), read as fp32
 *              (bf16 and fp16 convert exactly).
 *   threshold  position i is routed to full attention iff logits[i] >
 *              threshold (NaN never is).  For torch parity with
 *              `logits > t` on bf16/fp16 logits, pass t rounded to that
 *              dtype (torch compares in the tensor's dtype).
 *   indices, counts, workspace: as swattn_compact.
 */
#define SWATTN_DTYPE_F32 0
#define SWATTN_DTYPE_BF16 1
#define SWATTN_DTYPE_F16 2
int swattn_compact_logits(const void* logits, int32_t dtype, int64_t n, float threshold,
                          int32_t* indices, int32_t* counts, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * Index-list validation in one pass.  Replaces the device-side checks of
 * _prepare_indices (V:299-302, applied to both lists) and adds the
 * disjointness the docstring requires (V:341-342).  The count-based coverage
 * check (V:392-393) needs no device work and stays with the caller.
 *
 *   full/local  ascending int32 lists (n_full / n_local entries)
 *   seq_len     positions must lie in [0, seq_len)
 *   flags       1 int32 output: OR of SWATTN_ERR_* bits (0 = valid).
 * The caller reads `flags` back (one 4-byte device-to-host copy).
 */
int swattn_check_indices(const int32_t* full, int64_t n_full, const int32_t* local,
                         int64_t n_local, int64_t seq_len, int32_t* flags, void* stream);

/*
 * Position metadata for packed (varlen) sequences.  Replaces
 * build_switch_attention_metadata, imported by V:27 and called at V:353-359
 * but not shipped with the reference; the seven outputs are the fields the
 * wrapper validates at V:360-383 and the kernel reads at V:134-137.
 *
 *   cu_seqlens_q / cu_seqlens_kv  num_seqs+1 ascending int32 offsets (device)
 *   total_q / total_kv            cu_seqlens_*[num_seqs]
 *   outputs (int32, device):  q_positions[total_q], kv_positions[total_kv],
 *     q_segment_ids[total_q], kv_segment_ids[total_kv], full_starts[total_q],
 *     local_starts[total_q], causal_ends[total_q].
 * For query i (0-based inside its segment) with KV segment [ks, ke):
 *   full_starts = ks, local_starts = ks + max(i - window + 1, 0),
 *   causal_ends = ks + min(i + 1, ke - ks)      (F:145-155 per segment).
 */
int swattn_build_metadata(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kv,
                          int32_t num_seqs, int64_t total_q, int64_t total_kv, int32_t window,
                          int32_t* q_positions, int32_t* kv_positions, int32_t* q_segment_ids,
                          int32_t* kv_segment_ids, int32_t* full_starts, int32_t* local_starts,
                          int32_t* causal_ends, void* stream);

/*
 * Workspace bytes swattn_prefill_fwd needs for K/V of this shape (V is
 * repacked there as MFMA-ready V^T tiles); 0 for an unsupported shape.
 * No counterpart in the reference: its TileLang kernel reads V in place.
 */
size_t swattn_prefill_workspace_bytes(int32_t batch, int64_t seq_kv, int32_t heads_kv,
                                      int32_t head_dim);

/*
 * Workspace bytes that let swattn_prefill_fwd split long full-attention items
 * by key range; no counterpart in the reference, whose grid is one CTA per
 * query tile and head (V:402-445).  When the longest full item (a causal row
 * tile late in a sequence) is long against the rest of the work, as with few
 * KV heads (one GPU's share of a KV-head split) or short sequences on few
 * heads, a workgroup per chunk of key tiles (planned from the shape: 4 to 64
 * tiles, longer for very long sequences so that the chunk slots number at
 * most about 2048) and a merge of the chunks by their log2 LSE (V:236-241)
 * keep it from
 * setting the kernel's length.  Returns swattn_prefill_workspace_bytes() when
 * no split would run, a larger size (fp32 partial rows of the split items,
 * at most 200 MiB more) when it would, 0 for an unsupported shape.  The forward splits only if it
 * receives at least this much workspace; with less it runs unsplit.  Rows of
 * items that lie inside one chunk are computed exactly as without a split.
 */
size_t swattn_prefill_split_workspace_bytes(int32_t batch, int64_t seq_q, int64_t seq_kv,
                                            int32_t heads_q, int32_t heads_kv,
                                            int32_t head_dim, int32_t window, int64_t n_full,
                                            int64_t n_local);

/*
 * Routed GQA prefill forward, both branches in one launch.  Replaces the two
 * _switch_gqa_prefill_branch launches of switch_gqa_prefill_forward
 * (V:402-445; kernel body V:103-249, fixed-length rule F:69-214).
 *
 *   q    bf16 [batch, seq_q, heads_q, 128]   (contiguous)
 *   k,v  bf16 [batch, seq_kv, heads_kv, 128] (contiguous)
 *   full_idx / local_idx  ascending flattened row positions b*seq_q + i
 *                         (n_full + n_local rows, disjoint; pre-validated)
 *   full_starts, local_starts, causal_ends: per flattened query row key
 *        bounds in flattened key coordinates b*seq_kv + j; all three NULL
 *        selects F's rule (full: [0, i], local: [max(i-window+1, 0), i],
 *        both clipped to j < seq_kv) inside each batch row.
 *   out  bf16 [batch, seq_q, heads_q, 128], lse fp32 [batch, seq_q, heads_q]:
 *        rows listed in full_idx/local_idx are written; others untouched.
 *        lse uses the log2 convention: log2(sum_j 2^(s_j*c)) with
 *        c = scale_log2 and s_j the raw q.k products (V:236-241).
 *   scale_log2  softmax scale already multiplied by log2(e) (V:73-76).
 *   workspace   device scratch of at least swattn_prefill_workspace_bytes()
 *               (swattn_prefill_split_workspace_bytes() to allow the key-range
 *               split); overwritten by the call (calls sharing it must not
 *               overlap).
 */
int swattn_prefill_fwd(const void* q, const void* k, const void* v,
                       const int32_t* full_idx, int64_t n_full,
                       const int32_t* local_idx, int64_t n_local,
                       const int32_t* full_starts, const int32_t* local_starts,
                       const int32_t* causal_ends, void* out, float* lse,
                       int32_t batch, int64_t seq_q, int64_t seq_kv, int32_t heads_q,
                       int32_t heads_kv, int32_t head_dim, int32_t window, float scale_log2,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Split key ranges (context parallelism, ring passes).  No counterpart in the
 * reference, which covers the whole key range on one device; they build on
 * its log2 LSE export (V:15, V:236-241) and its split of query and key
 * positions in the metadata (V:139-141, V:179-182).
 *
 * swattn_shard_bounds: metadata bounds for query rows at global positions
 * q_positions[r] of one causal sequence against the key chunk
 * [kv_start, kv_end): the legal keys [0, p] (full) or [p - window + 1, p]
 * (local) (F:145-155), cut to the chunk and given in chunk coordinates
 * (key g -> g - kv_start).  A row with no key in the chunk gets an empty
 * range (start == end).  The three outputs feed swattn_prefill_fwd with K/V
 * pointing at the chunk.
 */
int swattn_shard_bounds(const int32_t* q_positions, int64_t n_q, int64_t kv_start, int64_t kv_end,
                        int32_t window, int32_t* full_starts, int32_t* local_starts,
                        int32_t* causal_ends, void* stream);

/*
 * swattn_merge_partials: combine n_parts (1..16) partial results over
 * disjoint key ranges into the result over their union:
 *   M = max_i LSE_i,  w_i = 2^(LSE_i - M),  LSE = M + log2(sum w_i),
 *   O = sum_i w_i O_i / sum_i w_i.
 * o_parts / lse_parts are host arrays of device pointers to bf16 [rows, 128]
 * and fp32 [rows] (rows = B*S*Hq; LSE in the log2 convention).  Parts with
 * LSE = -inf (no legal key) carry no weight; a row empty in every part is
 * written as O = NaN, LSE = -inf, like the attention kernel's empty rows.
 * out / lse_out may alias neither input.
 */
int swattn_merge_partials(const void* const* o_parts, const float* const* lse_parts,
                          int32_t n_parts, void* out, float* lse_out, int64_t rows,
                          int32_t head_dim, void* stream);

/*
 * Routed decode: one new query token per sequence attends its KV cache.  No
 * counterpart in the reference, which is prefill-only; the rule is the
 * prefill's for the last row (F:145-155): with len = cache_lens[b] (clamped
 * to [0, cache_len]) the token sits at position len - 1 and attends keys
 * [0, len) when full[b] != 0, else [max(len - window, 0), len).  Its own K/V
 * must already be in the cache at position len - 1.
 *
 *   q        bf16 [batch, heads_q, 128]
 *   k_cache, v_cache  bf16 [batch, cache_len, heads_kv, 128]
 *   cache_lens int32 [batch], full uint8 [batch]        (device)
 *   out      bf16 [batch, heads_q, 128], lse fp32 [batch, heads_q] (log2,
 *            V:236-241); a sequence with no key gets O = NaN, LSE = -inf.
 *   heads_q / heads_kv <= 8.  workspace >= swattn_decode_workspace_bytes(),
 *   which depends on the current device's CU count (ask on that device).
 * A one-workgroup plan kernel sizes key chunks on the device from the routed
 * key total (at least 256 keys, the same size for full and local
 * sequences); one workgroup per chunk; fp32 partials merged by a third kernel.
 */
size_t swattn_decode_workspace_bytes(int32_t batch, int64_t cache_len, int32_t heads_q,
                                     int32_t heads_kv);
int swattn_decode_fwd(const void* q, const void* k_cache, const void* v_cache,
                      const int32_t* cache_lens, const uint8_t* full, void* out, float* lse,
                      int32_t batch, int64_t cache_len, int32_t heads_q, int32_t heads_kv,
                      int32_t head_dim, int32_t window, float scale_log2, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * swattn_decode_fwd without a workspace: the one entry point that allocates
 * nothing and takes no scratch from the caller.  No counterpart in the
 * reference.  It is for callers that cannot allocate device memory: code
 * under HIP graph capture, tight serving loops, harnesses that forbid it.
 * Same arguments, kernels and results as swattn_decode_fwd.  Its scratch is
 * a library-owned device array of SWATTN_DECODE_NOALLOC_MAX_BYTES per GPU,
 * held until the process ends; a shape whose
 * swattn_decode_workspace_bytes() exceeds that is rejected (SWATTN_EINVAL,
 * with a message).  Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU (two streams, two threads) race and must be
 * serialised by the caller.  The first call on each device looks up that
 * device's array address (the device must be current, as for the launch).
 */
#define SWATTN_DECODE_NOALLOC_MAX_BYTES ((size_t)16 << 20)
int swattn_decode_fwd_noalloc(const void* q, const void* k_cache, const void* v_cache,
                              const int32_t* cache_lens, const uint8_t* full, void* out,
                              float* lse, int32_t batch, int64_t cache_len, int32_t heads_q,
                              int32_t heads_kv, int32_t head_dim, int32_t window,
                              float scale_log2, void* stream);

/*
 * Routed GQA prefill backward: dq, dk, dv of swattn_prefill_fwd's output.
 * No counterpart in the reference, which is forward-only (V:14-15); this is
 * the derivative of its forward (V:103-249) and consumes the log2 LSE it
 * exports (V:236-241).  For row r (query head h, KV head h / G) and legal
 * key j, with P = 2^(c q.k - LSE), Delta_r = dO_r . O_r and
 * dS = P (dO_r . v_j - Delta_r):
 *   dq_r = s sum_j dS k_j,  dk_j = s sum_r dS q_r,  dv_j = sum_r P dO_r,
 * s = sm_scale = scale_log2 * ln 2, dk/dv summed over the group's heads.
 *
 *   q, k, v, full_idx/local_idx, metadata, shapes, window, scale_log2: as
 *        passed to swattn_prefill_fwd (scale_log2 > 0).
 *   out, lse   that call's outputs (bf16 O, fp32 log2 LSE).
 *   dout       bf16 [batch, seq_q, heads_q, 128], the gradient of out.
 *   dq         bf16 like q: rows listed in full_idx/local_idx are written,
 *              others untouched; a row with no legal key gets 0.
 *   dk, dv     bf16 like k: every key row is written (0 where no row sees it).
 *   workspace  >= swattn_prefill_bwd_workspace_bytes(...): 1 KiB of row
 *              info per KV head and 32 listed rows, plus a little (Q and dO
 *              are read in place, never copied); for fewer than 512
 *              (256-key tile, KV head) pairs also fp32 dK/dV partials of
 *              256 KiB per split workgroup (at most 256 MiB), and, when the
 *              longest dQ row tile would set that pass's length, fp32 dQ
 *              partials of 128 KiB per piece slot (at most 192 MiB);
 *              overwritten (calls sharing it must not overlap).  The
 *              query takes the call's window to estimate the local rows'
 *              key ranges; pass the same shapes, window and list lengths
 *              to both.
 * Each list's key bounds must be non-decreasing along the list (true for
 * F:145-155 and for swattn_build_metadata / swattn_shard_bounds over
 * ascending positions): the keys a row block can see are found by a
 * search over them.
 */
size_t swattn_prefill_bwd_workspace_bytes(int32_t batch, int64_t seq_kv, int32_t heads_q,
                                          int32_t heads_kv, int32_t head_dim, int32_t window,
                                          int64_t n_full, int64_t n_local);
int swattn_prefill_bwd(const void* q, const void* k, const void* v, const void* out,
                       const float* lse, const void* dout, const int32_t* full_idx,
                       int64_t n_full, const int32_t* local_idx, int64_t n_local,
                       const int32_t* full_starts, const int32_t* local_starts,
                       const int32_t* causal_ends, void* dq, void* dk, void* dv, int32_t batch,
                       int64_t seq_q, int64_t seq_kv, int32_t heads_q, int32_t heads_kv,
                       int32_t head_dim, int32_t window, float scale_log2, void* workspace,
                       size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SWATTN_H_ */
