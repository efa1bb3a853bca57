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
 *   ssa_rep_values  <- the summary half of VR/csrc/fixed15_attention.cu:551-578
 *                      (prepare_fixed15: per-page summary tiles for the tail)
 *   ssa_route       <- VB/graph.py:102-211 BatchGraphs.compute (probe QK, risk,
 *                      quota_mask / base selection, final LUT) and
 *                      VR/legacy_components.py:14-22 risk(probes,z,summary,theta)
 */
#ifndef SSATTN_H
#define SSATTN_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Pre-projected rep values: rep_values[h,p,r,:] = bf16(mean[h,p,:] +
 * sum_k (sum_a HAAR[a,r] detail[h,p,a,k]) basis[h,:,k]) for p < pages.
 * mean [H,head_pages,128], detail [H,head_pages,3,8], basis [H,128,8] bf16;
 * rep_values [H,rep_head_pages,4,128] bf16. */
int ssa_rep_values(const void* mean, const void* detail, const void* basis, void* rep_values, int heads,
                   int pages, int head_pages, int rep_head_pages, hipStream_t stream);

/* One page-sparse attention call: exact attention over the `count` LUT pages
 * of each (query block, head) + compensation over the reps of the unselected
 * pages + softmax-mass merge, one fused kernel.
 * q, out [1,n_tokens,H,128] bf16 contiguous; k, v: page p, token j, head h at
 * element (64p+j)*kv_token_stride + h*kv_head_stride (+ dim); keys
 * [H,head_pages,4,128] bf16 (rep keys); rep_values from ssa_rep_values;
 * ids [H,n_tokens/64,count] int32 (page ids in [0,pages)).
 * flags bit 0: two-term bf16 P.V (hi + lo parts of each probability). */
int ssa_attention(const void* q, const void* k, const void* v, const void* keys, const void* rep_values,
                  const int32_t* ids, void* out, int n_tokens, int heads, int pages, int head_pages,
                  int rep_head_pages, int count, long long kv_token_stride, long long kv_head_stride, int flags,
                  hipStream_t stream);

/* Router: risk [H,blocks,pages] fp32 and, unless mode == -1, the page table.
 * Probe rows: gathered=1 -> q is probes [H,blocks,16,128] addressed
 * h*q_head_stride + t*q_block_stride + m*q_row_stride; gathered=0 -> q is the
 * query tensor and probe m of block t is query row 64t + offset[m] with
 * offsets {0,4,8,13,17,21,25,29,34,38,42,46,50,55,59,63}.
 * keys [H,head_pages,4,128] bf16, stats [H,head_pages,4,12] bf16, theta
 * [H,4] fp32, own [H,blocks] int32 or NULL (own = pages - blocks + t).
 * mode 0: base tier, ids = [own, 0..23, top count-25 by risk];
 * mode 1: anchor/current/history quota, current[h] = A >= 1, total = A+B,
 *         count = 24 + total, ids = own then selected by descending risk;
 * mode 2: fixed top-count with own forced first.  Ties -> lower page.
 * ids [H,blocks,count] int32 and mask [H,blocks,pages] uint8 may be NULL. */
int ssa_route(const void* q, long long q_head_stride, long long q_block_stride, long long q_row_stride,
              int gathered, const void* keys, const void* stats, const float* theta, const int32_t* current,
              const int32_t* own, float* risk, int32_t* ids, uint8_t* mask, int heads, int blocks, int pages,
              int head_pages, int count, int mode, int total, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SSATTN_H */
