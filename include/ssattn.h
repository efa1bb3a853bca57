/*
 * C ABI of libssattn.so: MI355X (gfx950) page-sparse streaming attention.
 *
 * All pointers are device addresses (e.g. torch.Tensor.data_ptr()), bf16
 * tensors are passed as raw 16-bit storage.  Every entry point enqueues work
 * on `stream`, allocates nothing, never synchronises, and returns a
 * hipError_t as int (0 = success; hipErrorInvalidValue = 1 for rejected
 * shapes).  Head dimension is fixed at 128; pages <= 512.
 *
 * Reference interfaces replaced (paths relative to jurky123/streaming_sparse,
 * VR = local_experiments/video_runtime_v1, RV = local_experiments/review_v1,
 * VB = reproduction/vbench_current):
 *   ssa_attention   <- VR/legacy_components.py:24-46 attention(q,k,v,s,basis,ids,
 *                      workspace,*,bf16_av) fused _tail path (RV/tuned_attention.py:
 *                      20-81) and the SM80 ctypes ABI `int run(...)`
 *                      (VR/csrc/fixed15_attention.cu:407-409, VR/fixed15_attention.py:13-32)
 *   ssa_rep_operands <- the summary half of VR/csrc/fixed15_attention.cu:551-578
 *                      (prepare_fixed15: per-page summary tiles for the tail)
 *   ssa_route       <- VB/graph.py:102-211 BatchGraphs.compute (probe QK, risk,
 *                      quota_mask / base selection, final LUT) and
 *                      VR/legacy_components.py:14-22 risk(probes,z,summary,theta)
 *   ssa_select      <- RV/ops.py:113-138 RouteOps.select(scores,own,config,
 *                      threshold,valid): counts, overflow, -1 padding, residual
 *   ssa_encode      <- VR/page.py:6-14 encode(summary,reader,phi,B) and
 *                      VideoRuntime.encode (VR/runtime.py:160-164)
 *   ssa_summary     <- the current-chunk summary recompute of VideoRuntime.forward
 *                      (VR/runtime.py:213-227; VR/summary_moments.py:113-137), with
 *                      k-means clusters as the token groups of RV/ops.py:43-76
 *   ssa_summary_write <- the same, fused with the window write of the chunk's
 *                      K/V before it (VR/runtime.py:205-206)
 *   ssa_pset        <- the Full_Pset branch of BatchGraphs.compute
 *                      (VB/graph.py:169-208): quota_pool.pool, read /
 *                      compact_scores (VR/page.py:17-21, VR/reader_reduce.py:150-190,
 *                      VR/scores.py:54-91), apply_best (VR/scores.py:102-107) and
 *                      the final LUT (VB/graph.py:210)
 */
#ifndef SSATTN_H
#define SSATTN_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Detail operand tiles of the compensation: for each head and each tile of
 * 16 pages (rt < ceil(pages/16)), 1024 bytes holding the detail rows
 * detail[h,p,a,:] (a = 0..2 Haar contrasts, rank 8) of the tile's pages in
 * the order the attention kernel's matrix products read them; pages >=
 * `pages` hold zeros.  detail [H,head_pages,3,8] bf16; rep_ops
 * [H,rep_tiles,512] bf16 (16-byte aligned), rep_tiles >= ceil(pages/16).
 * Recompute when the detail rows change. */
int ssa_rep_operands(const void* detail, void* rep_ops, int heads, int pages, int head_pages, int rep_tiles,
                     hipStream_t stream);

/* One page-sparse attention call: exact attention over the `count` LUT pages
 * of each (query block, head) + compensation over the reps of the unselected
 * pages + softmax-mass merge, one fused kernel.
 * q, out [1,n_tokens,H,128] bf16 contiguous; k, v: page p, token j, head h at
 * element (64p+j)*kv_token_stride + h*kv_head_stride (+ dim); keys
 * [H,head_pages,4,128] bf16 (rep keys); mean [H,head_pages,128] bf16 (page V
 * means); basis [H,128,8] bf16; rep_ops [H,rep_tiles,512] from
 * ssa_rep_operands (mean, basis and rep_ops 16-byte aligned; not read by a
 * dense call, flags bit 1);
 * ids [H,n_tokens/64,count] int32: page ids, own page first; entries
 * outside [0,pages) (the -1 padding of a shorter table, RV/ops.py:115) are
 * not read and select nothing; a page listed twice is attended twice.
 * flags bit 0: two-term bf16 products, the reference's HIGH_PRECISION_AV /
 * bf16_av=True arithmetic: the exact pages' P.V as bf16(P) V + bf16(P -
 * bf16(P)) V (LE/gap_exact_round_kernel.py:98-125), and in the compensation
 * the page-mean weights and the Haar contrast weights each as hi + lo bf16
 * parts against the bf16 mean and detail rows, as the tail's _av does
 * (RV/tuned_attention.py:16-18,60-62); the rank-8 code then meets the bf16
 * basis as a two-term bf16 product, where the reference's tail uses tf32x3
 * (RV/tuned_attention.py:71).  Clear: one bf16 term for every one of these
 * weights (single-term P.V).
 * flags bit 1: the caller guarantees every row of ids lists each page of the
 * window exactly once (count == pages, a dense call); ids are then not read
 * and two query blocks share each K/V page load.
 * flags bit 2: staged call (not with bit 1): the exact pages of every tile
 * in one launch, the compensation's rep tiles in a second, each leaving its
 * unnormalised softmax state in the workspace, then the merge kernel -- the
 * reference's split into an exact kernel, a tail and a merge
 * (RV/tuned_attention.py:20-81); the stages then show as separate kernels in
 * a profiler.  Needs the workspace (else hipErrorInvalidValue); results
 * agree with the fused call within its tolerance, not bit for bit.
 * workspace: device memory of workspace_bytes >= ssa_attention_workspace_bytes
 * of the same shape and flags (16-byte aligned; its contents on entry do
 * not matter), the stand-in for the reference's Workspace
 * (VR/attention.py:7-13).  With it, the
 * workgroups past the last multiple of the device's compute-unit count run
 * as pieces of their unit lists (two per (query block, head) tile in a
 * general call, four per two-block workgroup in a dense one), so the last
 * round spreads over every CU, and a second kernel merges the pieces'
 * states into out; NULL (or too small): every workgroup in one piece.  Results agree within the
 * call's tolerance, not bit for bit, between the two; each is
 * deterministic.  Calls that share a workspace must not overlap (one
 * stream, or ordered). */
int ssa_attention(const void* q, const void* k, const void* v, const void* keys, const void* mean, const void* basis,
                  const void* rep_ops, const int32_t* ids, void* out, int n_tokens, int heads, int pages,
                  int head_pages, int rep_tiles, int count, long long kv_token_stride, long long kv_head_stride,
                  int flags, void* workspace, long long workspace_bytes, hipStream_t stream);

/* Bytes of the ssa_attention workspace for a call of n_tokens queries,
 * heads heads, a window of pages pages and count table entries per row, with
 * these flags, on the current device (0: the call runs no split; -1:
 * invalid shape or flags, or no device).  The call's path (two-block dense
 * kernel, split, staged) follows from exactly these arguments, so the size
 * and the call agree.  No counterpart in the reference: its Workspace
 * allocates per call shape (VR/attention.py:7-13). */
long long ssa_attention_workspace_bytes(int n_tokens, int heads, int pages, int count, int flags);

/* Router: risk [H,blocks,pages] fp32 and, unless mode == -1, the page table.
 * Probe rows: gathered=1 -> q is probes [H,blocks,16,128] addressed
 * h*q_head_stride + t*q_block_stride + m*q_row_stride; gathered=0 -> q is the
 * query tensor and probe m of block t is query row 64t + offset[m] with
 * offsets {0,4,8,13,17,21,25,29,34,38,42,46,50,55,59,63}.
 * keys [H,head_pages,4,128] bf16, stats [H,head_pages,4,12] bf16 in the
 * reference's summary contract (RV/ops.py:66-75; slots 0..7 are mean squares,
 * >= 0, so the feature sqrt(max(u, 0)) is taken as sqrt(|u|)), theta
 * [H,4] fp32, own [H,blocks] int32 or NULL (own = pages - blocks + t).
 * mode 0: base tier, ids = [own, 0..23, top count-25 by risk];
 * mode 1: anchor/current/history quota (VB/quota_mask.py:7-39), total = A+B
 *         <= pages - 24, count = 24 + total: anchors 0..23, the top A of the
 *         current pages [pages-72, pages) with own forced, the top total-A
 *         of the history pages [24, pages-72), A = current[h]; each quota is
 *         clamped to [0, its partition's size] as the reference's _keep
 *         does (the history one computed from the unclamped A).
 *         pages == 72 (the anchor frame inside the chunk, VB/graph.py:
 *         143-148): anchors + the top `total` of pages [24,72), own forced;
 *         current may be NULL.  Otherwise pages >= 96.  ids = own first
 *         (also when its quota left it out), then the selected pages by
 *         descending risk, truncated to count, padded with -1;
 * mode 2: fixed top-count with own forced first.  Ties -> lower page.
 * own pages outside [0,pages) are clamped into the window.
 * ids [H,blocks,count] int32 and mask [H,blocks,pages] uint8 may be NULL; lse
 * [H,blocks,16] fp32 (NULL to skip) receives each probe's log-sum-exp over
 * all reps of the window (natural log), the input ssa_pset needs.
 * rep_ops [H,rep_tiles,512] bf16 (NULL to skip; 16-byte aligned, rep_tiles >=
 * ceil(pages/16)) receives, on the side, exactly what ssa_rep_operands
 * writes from detail [H,head_pages,3,8], so a call that routes needs no
 * separate operand launch.
 * Near-tie report (tie_rows NULL to skip; mode >= 0, tie_eps >= 0): the
 * rows h*blocks + t whose selection depends on a near tie are appended to
 * tie_rows [H*blocks] int32 in no particular order, and *tie_count (int32,
 * set to 0 by the call itself, graph-safe) receives their number -- the
 * compacted list and count of the reference's select_close / mark_close
 * (VR/csrc/risk_close.cu:35-79), which its recheck recomputes
 * (VR/risk_recheck.py:86-123).  A row is listed when, in a sorted run of
 * its selection (base: the pages >= 24 other than own, count-25 kept;
 * quota: the current pages with own first, A kept, and the history pages,
 * total-A kept, each clamped to the run; top-k: all pages with own first,
 * count kept), the last kept and the first dropped risks a, c (own, ranked
 * first by force, never counts) satisfy |a - c| <= tie_eps * max(|a|,
 * |c|). */
int ssa_route(const void* q, long long q_head_stride, long long q_block_stride, long long q_row_stride,
              int gathered, const void* keys, const void* stats, const float* theta, const int32_t* current,
              const int32_t* own, float* risk, int32_t* ids, uint8_t* mask, float* lse, int heads, int blocks,
              int pages, int head_pages, int count, int mode, int total, const void* detail, void* rep_ops,
              int rep_tiles, float tie_eps, int32_t* tie_rows, int32_t* tie_count, hipStream_t stream);

/* Measurement only, no counterpart in the reference: the phase stamps of the
 * last ssa_route launch, from the library built with -DSSA_ROUTE_STAMPS
 * (python -m streaming_sparse_amd.build --stamps -> libssattn_stamps.so).
 * Copies [1024 workgroups, 4 waves, 16] uint64 shader-clock stamps (lane 0
 * of each wave; slots 0..10 at the kernel's phase boundaries) into host
 * memory out of `bytes` >= 524288 and returns 0 after the copy; the product
 * library returns hipErrorNotSupported. */
int ssa_route_stamps(void* out, long long bytes);

/* Measurement only, no counterpart in the reference: the step stamps of the
 * last one-block attention launch (ssa_attention without the every-page
 * flag), from the same measurement build (-DSSA_ATTN_STAMPS).  Copies
 * [1024 workgroups, 4 waves, 296] uint64 into host memory out of `bytes` >=
 * 9699328 and returns 0 after the copy; the product library returns
 * hipErrorNotSupported.  A wave's record: 0 start, 1 unit list built,
 * 2 prologue done, 3 paired steps done, 4 last units done, 5 key halves
 * exchanged (shader clock, per XCD); 6 npages | nunits << 16 | ibeg << 32 |
 * (end of the paired steps) << 48; 7 HW_ID | XCC_ID << 32; then three clock
 * stamps per paired step k (unit ibeg + k, k < 96): step start, body done,
 * loads waited for. */
int ssa_attn_stamps(void* out, long long bytes);

/* Page selection from given scores (RV/ops.py:113-138 RouteOps.select), one
 * row per (head, block): scores [rows,pages] fp32, own [rows] int32, valid
 * [rows,pages] 0/1 bytes or NULL (all valid).  Pages rank with own first,
 * then valid pages by descending score (ties -> lower page), invalid pages
 * last.  use_threshold != 0: count = clamp(#(valid and score > threshold, own
 * counted), 1, cap) and overflow[row] = max(that number - cap, 0), with cap =
 * min(id_capacity, ceil(max_fraction * pages)) computed by the caller;
 * use_threshold == 0: count = min(fixed_count, #valid) (fixed_count =
 * max(1, floor(pages * density))) and overflow 0.  ids [rows,id_capacity]
 * int32: the first count ranked pages, then -1 (never to be read); counts
 * [rows] int32; mask [rows,pages] 0/1 bytes; residual [rows] fp32: the sum
 * of the scores of the valid unselected pages.  pages <= 512, 1 <= cap <=
 * min(id_capacity, pages). */
int ssa_select(const float* scores, const int32_t* own, const uint8_t* valid, int rows, int pages, float threshold,
               int use_threshold, int fixed_count, int cap, int id_capacity, int32_t* ids, int32_t* counts,
               uint8_t* mask, int32_t* overflow, float* residual, hipStream_t stream);

/* Page summaries of pages [first_page, first_page + pages) of the resident
 * cache (k, v addressed as in ssa_attention): a 4-way k-means of each page's
 * 64 keys from init [H, pages, 4] (token indices 0..63), `iters` >= 1 Lloyd
 * iterations (ties -> lower cluster), then keys [H,head_pages,4,128], mean
 * [H,head_pages,128], detail [H,head_pages,3,8], stats [H,head_pages,4,12]
 * (bf16) of those pages, with basis [H,128,8] bf16. */
int ssa_summary(const void* k, const void* v, long long kv_token_stride, long long kv_head_stride,
                const int32_t* init, const void* basis, void* keys, void* mean, void* detail, void* stats,
                int head_pages, int heads, int first_page, int pages, int iters, hipStream_t stream);

/* ssa_summary with the chunk's K/V written into the cache on the way:
 * page first_page + i of k, v (strides kv_*) receives rows 64 i .. 64 i + 63
 * of src_k, src_v (token stride src_token_stride, head stride
 * src_head_stride, in elements), and the summaries of those pages are
 * formed from the rows read.  Replaces the window write of the chunk's K/V
 * (key_window.copy_(k), value_window.copy_(v), VR/runtime.py:205-206)
 * followed by the summary recompute from k, v (VR/runtime.py:213-227): one
 * pass over the rows instead of a copy and a re-read.  Cache and summaries
 * equal a copy followed by ssa_summary, bit for bit.  src must not overlap
 * the cache pages it fills; sources and cache 16-byte aligned, strides
 * multiples of 8 elements. */
int ssa_summary_write(const void* src_k, const void* src_v, long long src_token_stride, long long src_head_stride,
                      void* k, void* v, long long kv_token_stride, long long kv_head_stride, const int32_t* init,
                      const void* basis, void* keys, void* mean, void* detail, void* stats, int head_pages,
                      int heads, int first_page, int pages, int iters, hipStream_t stream);

/* ssa_summary over `layers` (1..32) layers in one launch: k[l], v[l] (the
 * layer's cache, all with the same strides), basis[l] and the slab fields
 * keys[l], mean[l], detail[l], stats[l] (all with capacity head_pages) are
 * host arrays of the layers' device pointers; init, the page range and the
 * iterations are shared.  No counterpart in the reference, which summarises
 * layer by layer (the commit's VR/runtime.py:356-370, the anchor rebase's
 * VB/phase.py:4-25): for callers that refresh many layers at once.  Equal to
 * one ssa_summary per layer, bit for bit. */
int ssa_summary_layers(int layers, const void* const* k, const void* const* v, long long kv_token_stride,
                       long long kv_head_stride, const int32_t* init, const void* const* basis, void* const* keys,
                       void* const* mean, void* const* detail, void* const* stats, int head_pages, int heads,
                       int first_page, int pages, int iters, hipStream_t stream);

/* Full_Pset page encodings of pages [first_page, first_page + pages) of the
 * summary slab (keys/mean/detail/stats as in ssa_route, capacity head_pages):
 * coef [H,enc_pages,128] bf16 = co[85] (reader, [5,17]) | 11 zeros | A[32]
 * (phi, [8,4]); mean_b [H,enc_pages,16] and detail_b [H,enc_pages,3,16] fp64.
 * Weights fp32: w1t [712, 2*hidden] = both first layers transposed (columns
 * [0,hidden) reader, [hidden,2*hidden) phi), b1 [2*hidden]; w2_reader
 * [85,hidden], b2_reader [85]; w2_phi [32,hidden], b2_phi [32] (torch Linear
 * layout); B [128,16] fp64; basis [H,128,8] bf16.  hidden <= 256. */
int ssa_encode(const void* keys, const void* mean, const void* detail, const void* stats, int head_pages,
               const void* basis, const float* w1t, const float* b1, const float* w2_reader, const float* b2_reader,
               const float* w2_phi, const float* b2_phi, const double* B, void* coef, double* mean_b,
               double* detail_b, int enc_pages, int heads, int first_page, int pages, int hidden,
               hipStream_t stream);

/* ssa_encode over `layers` (1..32) layers in one launch: the slab fields,
 * the basis and the encodings coef, mean_b, detail_b are host arrays of the
 * layers' device pointers (equal capacities), the weights are shared.  No
 * counterpart in the reference, which encodes layer by layer
 * (VR/runtime.py:160-164 per layer): for callers that refresh many layers at
 * once.  Equal to one ssa_encode per layer, bit for bit. */
int ssa_encode_layers(int layers, const void* const* keys, const void* const* mean, const void* const* detail,
                      const void* const* stats, int head_pages, const void* const* basis, const float* w1t,
                      const float* b1, const float* w2_reader, const float* b2_reader, const float* w2_phi,
                      const float* b2_phi, const double* B, void* const* coef, double* const* mean_b,
                      double* const* detail_b, int enc_pages, int heads, int first_page, int pages, int hidden,
                      hipStream_t stream);

/* Full_Pset swap correction of the heads listed in heads[n_heads] (indices
 * into total_heads), after ssa_route in mode 1 produced risk, mask and ids.
 * Probe rows as in ssa_route; keys [H,head_pages,4,128] bf16; encodings from
 * ssa_encode; wq [8,128] fp32 (phi query map); probe_lse [H,blocks,16] from
 * ssa_route.  For each scoped (head, block)
 * the best legal same-partition swap is applied to mask [H,blocks,pages]
 * (0/1 bytes) iff its gain > 0 and every legal score is finite, and the row
 * of ids [H,blocks,count] is rebuilt (own first, then descending risk).
 * Caller-owned scratch: cand n_heads*blocks*16*48*34 fp64, rows
 * n_heads*blocks*16*2*52 fp64, pool n_heads*blocks*64 int32.  Per-row outputs:
 * gain [n_heads,blocks] fp64, info [n_heads,blocks,3] int32 = (executed, best
 * pair index remove*32+add, non-finite legal scores); scores
 * [n_heads,blocks,16,32] fp64 (illegal pairs -1e30) or NULL; stats [3]
 * int64 = (executed swaps, corrected rows, non-finite legal scores),
 * overwritten.
 * Pools: per partition (history [24,pages-72), current [pages-72,pages)),
 * up to 8 movable removes x 16 adds (VB/quota_pool.py:3-15,34-46); a
 * 72-page window (the first chunk, VB/quota_pool.py:21-33): up to 8 movable
 * removes (then the anchor pages other than own as stand-ins) x the first 16
 * of 32 adds (the unselected pages by descending risk, then the selected
 * pages in page order).
 * A padded add slot k takes the k-th page that is neither selected nor a
 * valid add; when there is none (the reference's pool indexes page P
 * there) the slot holds -1, an empty candidate of zero mass.
 * Requires pages == 72 with 24 <= count <= 72, or 96 < pages <= 512 with
 * 1 <= count <= pages. */
int ssa_pset(const void* q, long long q_head_stride, long long q_block_stride, long long q_row_stride,
             int gathered, const void* keys, int head_pages, const void* coef, const double* mean_b,
             const double* detail_b, int enc_pages, const float* wq, const float* risk, const float* probe_lse,
             uint8_t* mask, int32_t* ids, const int32_t* own, const int32_t* heads, int n_heads, double* cand,
             double* rows, int32_t* pool, double* gain, int32_t* info, double* scores, long long* stats,
             int total_heads, int blocks, int pages, int count, hipStream_t stream);

/* Anchor rebase (LE/anchor_rebase.py:8-18 shift_temporal_, as VB/phase.py:4-25
 * applies it to the cache's first frame): for `tokens` rows x `heads` of
 * 128-dim bf16 keys (src, dst addressed token*stride + head*stride + dim,
 * 4-byte aligned, even strides; dst may equal src), complex pair j < pairs
 * (dims 2j, 2j+1: the temporal RoPE pairs) is multiplied in fp64 by phase[j]
 * = (cos, sin) [pairs][2] (the rope table row of the offset) and rounded to
 * bf16 through fp32; the other dims are copied. */
int ssa_anchor_rebase(const void* src, long long src_token_stride, long long src_head_stride, void* dst,
                      long long dst_token_stride, long long dst_head_stride, const double* phase, int pairs,
                      int tokens, int heads, hipStream_t stream);

/* ssa_anchor_rebase over `layers` (1..32) layers in one launch: src[l] and
 * dst[l] are host arrays of the layers' device pointers (equal strides), the
 * phase is shared.  No counterpart in the reference, which rebases layer by
 * layer (VB/phase.py:4-25): for callers that rebase every layer at a chunk
 * boundary.  Equal to one ssa_anchor_rebase per layer, bit for bit. */
int ssa_anchor_rebase_layers(int layers, const void* const* src, long long src_token_stride,
                             long long src_head_stride, void* const* dst, long long dst_token_stride,
                             long long dst_head_stride, const double* phase, int pairs, int tokens, int heads,
                             hipStream_t stream);

/* Commit of a chunk's pages into the ring slots of the resident K/V cache
 * (RV/runtime.py:22-55 PageStore.commit / commit_indexed): row r of
 * destination page slots[p] (p < chunk_pages, slots[p] < dst_pages) takes
 * chunk token order[h, 64p + r] (order [H, 64 chunk_pages] int32, NULL: token
 * 64p + r) of head h, for K and V (token-major [tokens, H, 128] sources,
 * destinations addressed like ssa_attention's k/v; 16-byte aligned).  The
 * sources must not overlap the destination rows. */
int ssa_commit_pages(const void* k_src, const void* v_src, long long src_token_stride, long long src_head_stride,
                     const int32_t* order, int chunk_pages, const int32_t* slots, int dst_pages, void* k_dst,
                     void* v_dst, long long dst_token_stride, long long dst_head_stride, int heads,
                     hipStream_t stream);

/* ssa_commit_pages over `layers` (1..32) layers in one launch: k_src[l],
 * v_src[l], order[l] (NULL entries: token order), k_dst[l], v_dst[l] are host
 * arrays of the layers' device pointers (equal strides), the slots are
 * shared.  No counterpart in the reference, which commits layer by layer
 * (VR/runtime.py:356-370): for callers that commit every layer at the clean
 * step.  Equal to one ssa_commit_pages per layer, bit for bit. */
int ssa_commit_pages_layers(int layers, const void* const* k_src, const void* const* v_src,
                            long long src_token_stride, long long src_head_stride, const int32_t* const* order,
                            int chunk_pages, const int32_t* slots, int dst_pages, void* const* k_dst,
                            void* const* v_dst, long long dst_token_stride, long long dst_head_stride, int heads,
                            hipStream_t stream);

/* Clean-commit token grouping (RV/runtime.py:57-68 GroupingOps.group with the
 * features of LE/all_sparse_model.py:16-23, LE/response_hard.py:20-31
 * balanced splits 3,3,2,2,2 then 2,2 inside each page, the page order of
 * RV/ops.py:25-28 and, with first_chunk, the stable re-sort by frame of
 * VR/runtime.py:358-363), in fp64 from the bf16 inputs.  For each of
 * layers x heads rows b = layer*heads + head: k, v are the chunk's 4608
 * tokens (element layer*layer_stride + token*token_stride + head*head_stride
 * + dim), bank [B,32,128], group_v [B,128,32], gate [B,32] fp32, page_dst
 * [72] (destination page of grouped page p, NULL: identity).  order [B,4608]
 * int32 receives the chunk token of each destination position (the `order`
 * ssa_commit_pages takes).  k, v, bank and group_v 16-byte aligned, strides
 * multiples of 8 elements.  Scratch: scratch_x 2*B*4608*32 fp64,
 * scratch_ids 2*B*4608 int32. */
int ssa_group_order(const void* k, const void* v, long long layer_stride, long long token_stride,
                    long long head_stride, const float* bank, const float* group_v, const float* gate,
                    const int32_t* page_dst, int first_chunk, int layers, int heads, double* scratch_x,
                    int32_t* scratch_ids, int32_t* order, hipStream_t stream);

/* ssa_pset without the caller-owned scratch (cand, rows, pool): the library
 * keeps that scratch in a file-scope device array of 48.05 MB per device
 * (held until the process ends), sized for n_heads * blocks <= 216 scoped rows
 * (3 heads x 72 query blocks); larger calls return hipErrorInvalidValue.
 * Allocates nothing (no hipMalloc, no allocating library routine); the first
 * call on a device looks the array's device address up.  Every call on one
 * device shares that array: calls that overlap on one device race.
 * No counterpart in the reference: this entry point is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  Other arguments and results as in
 * ssa_pset. */
int ssa_pset_noalloc(const void* q, long long q_head_stride, long long q_block_stride, long long q_row_stride,
                     int gathered, const void* keys, int head_pages, const void* coef, const double* mean_b,
                     const double* detail_b, int enc_pages, const float* wq, const float* risk,
                     const float* probe_lse, uint8_t* mask, int32_t* ids, const int32_t* own, const int32_t* heads,
                     int n_heads, double* gain, int32_t* info, double* scores, long long* stats, int total_heads,
                     int blocks, int pages, int count, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SSATTN_H */
