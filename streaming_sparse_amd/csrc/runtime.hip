// Device work of the rolling KV window around the attention call:
//   * anchor rebase: the anchor frame's keys re-rotated so the current frames
//     sit at a fixed temporal distance (LE/anchor_rebase.py:8-18,
//     VB/phase.py:4-25);
//   * commit: a chunk's 72 pages (tokens in the grouped order) written into
//     the ring slots of the resident K/V cache (RV/runtime.py:22-55).
// Both are HBM-bound copies with a little arithmetic per element.
#include "common.h"

using namespace ssa;

namespace {

constexpr int kPairsPerRow = kHeadDim / 2;   // complex pairs of one key row

// Per-layer tensors of a batched launch (blockIdx.z = layer); a one-layer
// launch passes its tensors as entry 0.
constexpr int kMaxLayers = 32;
struct RebaseLayers {
  const uint16_t* src[kMaxLayers];
  uint16_t* dst[kMaxLayers];
};
struct CommitLayers {
  const uint16_t *k_src[kMaxLayers], *v_src[kMaxLayers];
  const int32_t* order[kMaxLayers];
  uint16_t *k_dst[kMaxLayers], *v_dst[kMaxLayers];
};

// fp64 -> bf16 as a float64 tensor's .to(bfloat16) does it: round to fp32
// first, then round-to-nearest-even to bf16 on the fp32 bits (finite
// values).  The integer step keeps the compiler from folding the two
// roundings into one.
__device__ __forceinline__ uint32_t f64_to_bf16(double x) {
  const uint32_t u = __float_as_uint((float)x);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// One thread per complex pair (token, head, pair): pairs j < `pairs` (the
// temporal RoPE components) are multiplied by phase[j] = cos + i sin in
// fp64 -- (a c - b d) + i (a d + b c), each product and sum rounded on its
// own (no fused multiply-add), as a complex128 product is -- and rounded to
// bf16; the other pairs (spatial components) are copied bit for bit.
// Grid: (tokens, ceil(heads * 64 / 256)).
__global__ __launch_bounds__(256) void anchor_rebase_kernel(RebaseLayers layers, long long src_tok,
                                                            long long src_head, long long dst_tok,
                                                            long long dst_head, const double* phase, int pairs,
                                                            int heads) {
#pragma clang fp contract(off)
  const uint16_t* src = layers.src[blockIdx.z];
  uint16_t* dst = layers.dst[blockIdx.z];
  const int hp = blockIdx.y * blockDim.x + threadIdx.x;
  if (hp >= heads * kPairsPerRow) return;
  const int h = hp / kPairsPerRow, j = hp % kPairsPerRow;
  const long long t = blockIdx.x;
  const uint32_t w = *reinterpret_cast<const uint32_t*>(src + t * src_tok + h * src_head + 2 * j);
  uint32_t out = w;
  if (j < pairs) {
    const double a = (double)bf16_lo(w), b = (double)bf16_hi(w);
    const double c = phase[2 * j], d = phase[2 * j + 1];
    const double ac = a * c, bd = b * d, ad = a * d, bc = b * c;
    out = f64_to_bf16(ac - bd) | (f64_to_bf16(ad + bc) << 16);
  }
  *reinterpret_cast<uint32_t*>(dst + t * dst_tok + h * dst_head + 2 * j) = out;
}

// One workgroup per (chunk page, head): destination row r of ring page
// slots[page] takes source token order[h, 64 page + r] (order null: 64 page
// + r) of the chunk, K and V.  16 threads move one 256-byte row.
__global__ __launch_bounds__(256) void commit_pages_kernel(CommitLayers layers, long long src_tok,
                                                           long long src_head, int chunk_tokens,
                                                           const int32_t* slots, int dst_pages, long long dst_tok,
                                                           long long dst_head, int heads) {
  const int page = blockIdx.x, h = blockIdx.y, l = blockIdx.z;
  const uint16_t *k_src = layers.k_src[l], *v_src = layers.v_src[l];
  const int32_t* order = layers.order[l];
  uint16_t *k_dst = layers.k_dst[l], *v_dst = layers.v_dst[l];
  const int tid = threadIdx.x, c = tid & 15;
  // slots and order entries are clamped into their ranges (memory safety;
  // valid inputs are inside them)
  const long long base = (long long)min(max(slots[page], 0), dst_pages - 1) * 64;
  for (int r = tid >> 4; r < 64; r += 16) {
    const int j = page * 64 + r;
    const int s = order ? min(max(order[(long long)h * chunk_tokens + j], 0), chunk_tokens - 1) : j;
    const long long so = (long long)s * src_tok + (long long)h * src_head + 8 * c;
    const long long dofs = (base + r) * dst_tok + (long long)h * dst_head + 8 * c;
    *reinterpret_cast<u32x4*>(k_dst + dofs) = ldg16(k_src + so);
    *reinterpret_cast<u32x4*>(v_dst + dofs) = ldg16(v_src + so);
  }
}

int rebase_launch(int layers, const void* const* src, long long src_token_stride, long long src_head_stride,
                  void* const* dst, long long dst_token_stride, long long dst_head_stride, const double* phase,
                  int pairs, int tokens, int heads, hipStream_t stream) {
  if (layers < 1 || layers > kMaxLayers || tokens <= 0 || heads <= 0 || pairs < 0 || pairs > kPairsPerRow ||
      (pairs > 0 && phase == nullptr) || src == nullptr || dst == nullptr || src_token_stride < 0 ||
      src_head_stride < 0 || dst_token_stride < 0 || dst_head_stride < 0)
    return (int)hipErrorInvalidValue;
  // 4-byte pair loads and stores
  if ((src_token_stride | src_head_stride | dst_token_stride | dst_head_stride) & 1) return (int)hipErrorInvalidValue;
  if (heads > 4096) return (int)hipErrorInvalidValue;
  RebaseLayers t;
  for (int l = 0; l < layers; ++l) {
    if (src[l] == nullptr || dst[l] == nullptr || (((uintptr_t)src[l] | (uintptr_t)dst[l]) & 3))
      return (int)hipErrorInvalidValue;
    t.src[l] = (const uint16_t*)src[l];
    t.dst[l] = (uint16_t*)dst[l];
  }
  hipLaunchKernelGGL(anchor_rebase_kernel, dim3(tokens, (heads * kPairsPerRow + 255) / 256, layers), dim3(256), 0,
                     stream, t, src_token_stride, src_head_stride, dst_token_stride, dst_head_stride, phase, pairs,
                     heads);
  return (int)hipGetLastError();
}

int commit_launch(int layers, const void* const* k_src, const void* const* v_src, long long src_token_stride,
                  long long src_head_stride, const int32_t* const* order, int chunk_pages, const int32_t* slots,
                  int dst_pages, void* const* k_dst, void* const* v_dst, long long dst_token_stride,
                  long long dst_head_stride, int heads, hipStream_t stream) {
  if (layers < 1 || layers > kMaxLayers || chunk_pages <= 0 || heads <= 0 || dst_pages <= 0 || slots == nullptr ||
      !k_src || !v_src || !order || !k_dst || !v_dst)
    return (int)hipErrorInvalidValue;
  // 16-byte row pieces
  if ((src_token_stride | src_head_stride | dst_token_stride | dst_head_stride) & 7) return (int)hipErrorInvalidValue;
  CommitLayers t;
  for (int l = 0; l < layers; ++l) {
    if (!k_src[l] || !v_src[l] || !k_dst[l] || !v_dst[l] ||
        (((uintptr_t)k_src[l] | (uintptr_t)v_src[l] | (uintptr_t)k_dst[l] | (uintptr_t)v_dst[l]) & 15))
      return (int)hipErrorInvalidValue;
    t.k_src[l] = (const uint16_t*)k_src[l];
    t.v_src[l] = (const uint16_t*)v_src[l];
    t.order[l] = order[l];
    t.k_dst[l] = (uint16_t*)k_dst[l];
    t.v_dst[l] = (uint16_t*)v_dst[l];
  }
  hipLaunchKernelGGL(commit_pages_kernel, dim3(chunk_pages, heads, layers), dim3(256), 0, stream, t,
                     src_token_stride, src_head_stride, chunk_pages * 64, slots, dst_pages, dst_token_stride,
                     dst_head_stride, heads);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

int ssa_anchor_rebase(const void* src, long long src_token_stride, long long src_head_stride, void* dst,
                      long long dst_token_stride, long long dst_head_stride, const double* phase, int pairs,
                      int tokens, int heads, hipStream_t stream) {
  return rebase_launch(1, &src, src_token_stride, src_head_stride, &dst, dst_token_stride, dst_head_stride, phase,
                       pairs, tokens, heads, stream);
}

int ssa_anchor_rebase_layers(int layers, const void* const* src, long long src_token_stride,
                             long long src_head_stride, void* const* dst, long long dst_token_stride,
                             long long dst_head_stride, const double* phase, int pairs, int tokens, int heads,
                             hipStream_t stream) {
  return rebase_launch(layers, src, src_token_stride, src_head_stride, dst, dst_token_stride, dst_head_stride, phase,
                       pairs, tokens, heads, stream);
}

int ssa_commit_pages(const void* k_src, const void* v_src, long long src_token_stride, long long src_head_stride,
                     const int32_t* order, int chunk_pages, const int32_t* slots, int dst_pages, void* k_dst,
                     void* v_dst, long long dst_token_stride, long long dst_head_stride, int heads,
                     hipStream_t stream) {
  return commit_launch(1, &k_src, &v_src, src_token_stride, src_head_stride, &order, chunk_pages, slots, dst_pages,
                       &k_dst, &v_dst, dst_token_stride, dst_head_stride, heads, stream);
}

int ssa_commit_pages_layers(int layers, const void* const* k_src, const void* const* v_src,
                            long long src_token_stride, long long src_head_stride, const int32_t* const* order,
                            int chunk_pages, const int32_t* slots, int dst_pages, void* const* k_dst,
                            void* const* v_dst, long long dst_token_stride, long long dst_head_stride, int heads,
                            hipStream_t stream) {
  return commit_launch(layers, k_src, v_src, src_token_stride, src_head_stride, order, chunk_pages, slots, dst_pages,
                       k_dst, v_dst, dst_token_stride, dst_head_stride, heads, stream);
}

}  // extern "C"
