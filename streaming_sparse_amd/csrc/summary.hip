// Page summaries on gfx950: a seeded 4-way k-means of each page's 64 keys
// (4 Lloyd iterations) and the reference's summary contract built on it.
//
// Per page of one head (RV/ops.py:43-76 with the learned pooling replaced by
// k-means clusters as the token groups):
//   keys   pk_r = bf16(km_r - mean_r km + mean_t k)        (RV/ops.py:60)
//   mean   mu   = bf16(mean_t v)                           (RV/ops.py:61)
//   detail bf16(sum_r HAAR[a,r] (vm_r . bf16(basis)) / 4)  (RV/ops.py:63-64)
//   stats  [r, 0:8] mean over 16-dim groups of the cluster key variance,
//          [r, 8] |km_r - pk_r|, [r, 9] |vm_r - recon_r|, [r, 10] V spread,
//          [0, 11] |mean v - mu|, [1, 11] max_t |v_t|      (RV/ops.py:66-75)
// where km_r / vm_r are the cluster key / value means (an empty cluster
// keeps its centroid and takes the page V mean).
//
// One workgroup (256 threads, 4 waves) per (page, head).  Thread (token
// t = lane, quarter q = wave) keeps dims 32q..32q+31 of its key in registers
// for the distance passes; the page's K and V are also staged in LDS as bf16
// pairs.  The cluster sums of each Lloyd step (and the page and cluster V
// sums after the last) run on the matrix pipe: wave w forms out[cluster][dim]
// = M^T . rows for dims 32w..32w+31, with the 0/1 membership M built from
// the wave-uniform member masks and the rows read by LDS transpose reads; a
// sum of at most 64 bf16 values is exact in fp32 whenever their exponents
// span no more than 10 binades, so it does not depend on the order of the
// additions.  The key variances and the V spread, thread (cluster r = wave,
// dims 2 lane, 2 lane + 1), accumulate over the cluster's member tokens in
// ascending token order.  LDS stays under 40 KB so four workgroups share a
// CU.
//
// ssa_summary_write reads the page rows from the chunk's K/V instead and
// writes them into the cache in the same pass (the window write that
// precedes the summary recompute, VR/runtime.py:205-206).
#include "common.h"

#include <type_traits>

using namespace ssa;

namespace {

constexpr float kHaar[3][4] = {{1, 1, -1, -1}, {1, -1, 1, -1}, {1, -1, -1, 1}};

struct SummaryParams {
  const uint16_t *k, *v;
  long long kv_tok, kv_head;
  // write-through (src_k non-null): page pl's 64 rows are read from
  // src_k / src_v tokens 64 pl .. 64 pl + 63 and written to the cache
  // (k, v) at page first + pl before the summary is formed from them
  const uint16_t *src_k, *src_v;
  long long src_tok, src_head;
  const int32_t* init;          // [H, pages, 4] initial tokens
  const uint16_t* basis;        // [H, 128, 8]
  uint16_t *keys, *mean, *detail, *stats;
  int HP, first, pages, iters;
};

// Per-layer tensors of a batched call (blockIdx.z = layer): the cache, the
// basis and the summary slab of each layer; everything else is shared.
constexpr int kMaxLayers = 32;
struct SummaryLayers {
  const uint16_t *k[kMaxLayers], *v[kMaxLayers], *basis[kMaxLayers];
  uint16_t *keys[kMaxLayers], *mean[kMaxLayers], *detail[kMaxLayers], *stats[kMaxLayers];
};
struct OneLayer {};

struct SumSmem {
  // row t = token, 64 words (bf16 pairs); 16 B chunk c of row t sits at
  // chunk c ^ (t & 15), so both the row-wise 16 B writes and the per-word
  // column walks are bank-conflict free
  alignas(16) uint32_t K[64 * 64];
  alignas(16) uint32_t V[64 * 64];
  alignas(16) float cent[4][128];
  union {
    f32x4 dist[4][64];                 // [quarter][token] partial distances to the 4 centroids
    float vnp[4][64];                  // [quarter][token] partial |v|^2 (before the first distance pass)
    float vm[4][128];                  // [cluster][dim] cluster V means (after the last assignment)
  } u;
  float kmean[128], vmean[128];
  float code[4][8];
};

__device__ __forceinline__ int word(int t, int w) { return t * 64 + (w ^ ((t & 15) << 2)); }

__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce(v, [](float a, float b) { return a + b; });
}

// Words `lane` of the K and V rows of the next kWalk member tokens of m
// (removed from m), in ascending token order.  The token ids come from the
// wave-uniform mask without branches and every read is issued before the
// first use; a slot past the last member re-reads token 0, which the caller
// does not accumulate.
constexpr int kWalk = 8;
__device__ __forceinline__ void next_members(const uint32_t* krows, const uint32_t* vrows, uint64_t& m, int lane,
                                             uint32_t (&wk)[kWalk], uint32_t (&wv)[kWalk]) {
#pragma unroll
  for (int u = 0; u < kWalk; ++u) {
    const int t = m ? __builtin_ctzll(m) : 0;
    m &= m - 1;
    wk[u] = krows[word(t, lane)];
    wv[u] = vrows[word(t, lane)];
  }
}

typedef __attribute__((address_space(3))) const uint8_t lds_u8;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// B operand of the cluster sums: the page rows (K or V) at dims
// 32 dt + lane % 32 for the tokens 16 ks + 8 (e / 4) + 4 (lane / 32) + e % 4
// of its 8 elements e, by two LDS transpose reads (ds_read_b64_tr_b16) of the
// token-major rows.
__device__ __forceinline__ u32x4 rows_operand(const uint32_t* rows, int dt, int ks, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int chunk = 4 * dt + 2 * (g & 1) + ((i & 3) >> 1);
  const int r0 = 16 * ks + 4 * (g >> 1) + (i >> 2), r1 = r0 + 8;
  const lds_u8* base = (const lds_u8*)rows + (i & 1) * 8;
  const bf16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(base + r0 * 256 + ((chunk ^ (r0 & 15)) << 4)));
  const bf16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(base + r1 * 256 + ((chunk ^ (r1 & 15)) << 4)));
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return u32x4{ua[0], ua[1], ub[0], ub[1]};
}

// A operand of the cluster sums: row m = lane % 32 is the 0/1 membership of
// cluster m (m < 4) or all ones (m == 4: the page sum) or zero, over the
// tokens of rows_operand's k order.
__device__ __forceinline__ u32x4 member_operand(const uint64_t (&mk)[4], int ks, int lane) {
  const int m = lane & 31, hh = lane >> 5;
  const uint64_t msk = m < 4 ? mk[m] : (m == 4 ? ~0ull : 0ull);
  const uint32_t bits = (uint32_t)((msk >> (16 * ks + 4 * hh)) & 0xFu) |
                        ((uint32_t)((msk >> (16 * ks + 8 + 4 * hh)) & 0xFu) << 4);
  u32x4 w;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = ((bits >> (2 * j)) & 1u ? 0x3F80u : 0u) | ((bits >> (2 * j + 1)) & 1u ? 0x3F800000u : 0u);
  return w;
}

// Sums over the member tokens of each cluster (and over the whole page) of
// dims 32 dt .. 32 dt + 31 of the rows: out[cluster][dim] = M^T . rows on
// v_mfma_f32_32x32x16_bf16 (fp32 sums of bf16 values times 1).  Lane l < 32
// gets the 4 cluster sums of dim 32 dt + l in items 0..3, lane l + 32 the
// page sum of that dim in item 0.
__device__ __forceinline__ f32x16 cluster_sums(const uint32_t* rows, const uint64_t (&mk)[4], int dt, int lane) {
  f32x16 c = {};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) c = mfma32(member_operand(mk, ks, lane), rows_operand(rows, dt, ks, lane), c);
  return c;
}

template <class Layers>
__global__ __launch_bounds__(256, 4) void summary_kernel(SummaryParams p, Layers layers) {
  if constexpr (std::is_same_v<Layers, SummaryLayers>) {
    const int l = blockIdx.z;
    p.k = layers.k[l];
    p.v = layers.v[l];
    p.basis = layers.basis[l];
    p.keys = layers.keys[l];
    p.mean = layers.mean[l];
    p.detail = layers.detail[l];
    p.stats = layers.stats[l];
  }
  __shared__ SumSmem s;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pl = blockIdx.x, h = blockIdx.y;
  const int page = p.first + pl;
  const long long base = (long long)page * 64 * p.kv_tok + (long long)h * p.kv_head;
  const int d0 = 2 * lane, d1 = 2 * lane + 1;
  // global reads up front: this thread's key/value quarter, its two basis
  // rows, the initial token of centroid `wave`
  const int init_tok = p.init[((long long)h * p.pages + pl) * 4 + wave] & 63;
  float bas0[8], bas1[8];
  {
    const u32x4 b0 = ldg16(p.basis + (long long)h * 1024 + d0 * 8);
    const u32x4 b1 = ldg16(p.basis + (long long)h * 1024 + d1 * 8);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      bas0[2 * w] = bf16_lo(b0[w]);
      bas0[2 * w + 1] = bf16_hi(b0[w]);
      bas1[2 * w] = bf16_lo(b1[w]);
      bas1[2 * w + 1] = bf16_hi(b1[w]);
    }
  }
  // The page's K and V rows reach LDS by row-coalesced 1 KB DMA loads (wave
  // w: rows 16 w .. 16 w + 15, 4 rows per load, each lane one 16-byte chunk
  // at its swizzled place); a load in which every lane read a piece of its
  // own token's row would cost the address unit 64 rows per instruction.
  const uint16_t* ksrc = p.src_k ? p.src_k + (long long)pl * 64 * p.src_tok + (long long)h * p.src_head : p.k + base;
  const uint16_t* vsrc = p.src_k ? p.src_v + (long long)pl * 64 * p.src_tok + (long long)h * p.src_head : p.v + base;
  const long long stok = p.src_k ? p.src_tok : p.kv_tok;
  {
    const uint32_t kl = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)s.K);
    const uint32_t vl = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)s.V);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int r = 16 * wave + 4 * jj + (lane >> 4);
      const uint32_t off = (uint32_t)(2 * (r * stok + 8 * ((lane & 15) ^ (r & 15))));
      const uint32_t dst = (uint32_t)((16 * wave + 4 * jj) * 256);
      dma16(ksrc, off, kl + dst);
      dma16(vsrc, off, vl + dst);
    }
  }
  wait_loads();
  __syncthreads();
  if (p.src_k) {
    // write-through: the same rows into the window, 4 rows per store
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int r = 16 * wave + 4 * jj + (lane >> 4), c = lane & 15;
      const int at = r * 64 + 4 * (c ^ (r & 15));
      const long long dst = base + (long long)r * p.kv_tok + 8 * c;
      *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(p.k) + dst) = *reinterpret_cast<const u32x4*>(&s.K[at]);
      *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(p.v) + dst) = *reinterpret_cast<const u32x4*>(&s.V[at]);
    }
  }
  // thread (token lane, quarter wave): dims 32 wave .. 32 wave + 31 of its
  // key in registers for the distance passes, and its share of |v|^2
  float kr[32];
  {
    float vn = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int chunk = (4 * wave + j) ^ (lane & 15);
      const u32x4 a = *reinterpret_cast<const u32x4*>(&s.K[lane * 64 + 4 * chunk]);
      const u32x4 b = *reinterpret_cast<const u32x4*>(&s.V[lane * 64 + 4 * chunk]);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        kr[8 * j + 2 * w] = bf16_lo(a[w]);
        kr[8 * j + 2 * w + 1] = bf16_hi(a[w]);
        const float x0 = bf16_lo(b[w]), x1 = bf16_hi(b[w]);
        vn = fmaf(x0, x0, vn);
        vn = fmaf(x1, x1, vn);
      }
    }
    s.u.vnp[wave][lane] = vn;
  }
  __syncthreads();
  // initial centroids, max token |v| (wave 1 keeps it)
  {
    const uint32_t w = s.K[word(init_tok, lane)];
    s.cent[wave][d0] = bf16_lo(w);
    s.cent[wave][d1] = bf16_hi(w);
  }
  float vmax = 0.f;
  if (wave == 1) {
    vmax = sqrtf(((s.u.vnp[0][lane] + s.u.vnp[1][lane]) + s.u.vnp[2][lane]) + s.u.vnp[3][lane]);
    vmax = wave_reduce(vmax, [](float a, float b) { return fmaxf(a, b); });
  }
  __syncthreads();

  // Lloyd iterations: assign each token to its nearest centroid (squared
  // distance, ties -> lower cluster), then move every non-empty centroid to
  // its cluster mean.  An assignment equal to the previous one is a fixed
  // point: the update would rebuild the same centroids from the same member
  // sums, and every later iteration would repeat both, so the loop ends
  // there with the result of all p.iters iterations, bit for bit.
  uint64_t memb[4] = {0, 0, 0, 0};   // member tokens of each cluster (wave-uniform)
  for (int it = 0; it < p.iters; ++it) {
    float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const f32x4 c = *reinterpret_cast<const f32x4*>(&s.cent[r][32 * wave + 4 * j]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = kr[4 * j + e] - c[e];
          d[r] = fmaf(x, x, d[r]);
        }
      }
    }
    s.u.dist[wave][lane] = f32x4{d[0], d[1], d[2], d[3]};
    __syncthreads();
    // every wave: token lane's distances over the 4 quarters, nearest centroid
    f32x4 tot = s.u.dist[0][lane];
#pragma unroll
    for (int q = 1; q < 4; ++q) tot += s.u.dist[q][lane];
    int best = 0;
    float bv = tot[0];
#pragma unroll
    for (int r = 1; r < 4; ++r) {
      if (tot[r] < bv) {
        bv = tot[r];
        best = r;
      }
    }
    uint64_t nm[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) nm[r] = __ballot(best == r);
    // every wave forms the same assignment from the same distances, so the
    // exit is uniform; the barrier keeps the distance slots (a union with
    // the cluster V means written next) until every wave has read them
    if (it > 0 && nm[0] == memb[0] && nm[1] == memb[1] && nm[2] == memb[2] && nm[3] == memb[3]) {
      __syncthreads();
      break;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) memb[r] = nm[r];
    // the cluster sums of dims 32 wave .. 32 wave + 31 (and the page sum, on
    // the first pass) on the matrix pipe; lane l < 32 then holds the 4
    // cluster sums of dim 32 wave + l, lane l + 32 its page sum
    const f32x16 cs = cluster_sums(s.K, memb, wave, lane);
    if (lane < 32) {
      const int d = 32 * wave + lane;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (memb[r]) s.cent[r][d] = cs[r] / (float)__popcll(memb[r]);
    } else if (it == 0) {
      s.kmean[32 * wave + lane - 32] = cs[0] / 64.f;
    }
    __syncthreads();
  }
  const uint64_t mr = memb[wave];   // member tokens of cluster `wave`
  // the cluster V means of dims 32 wave .. 32 wave + 31 (an empty cluster
  // takes the page V mean), through LDS to the threads of each cluster
  {
    const f32x16 cs = cluster_sums(s.V, memb, wave, lane);
    const float page = __shfl_xor(cs[0], 32);
    if (lane < 32) {
      const int d = 32 * wave + lane;
      const float vmean = page / 64.f;
      s.vmean[d] = vmean;
#pragma unroll
      for (int r = 0; r < 4; ++r) s.u.vm[r][d] = memb[r] ? cs[r] / (float)__popcll(memb[r]) : vmean;
    }
  }
  __syncthreads();

  // thread (cluster r = wave, dims 2 lane, 2 lane + 1): key variance and V
  // spread over the cluster's member tokens, in ascending token order
  const int r = wave;
  const int cnt = __popcll(mr);
  const float div = (float)max(cnt, 1);
  const float c0 = s.cent[r][d0], c1 = s.cent[r][d1];
  const float vm0 = s.u.vm[r][d0], vm1 = s.u.vm[r][d1];
  float var0 = 0.f, var1 = 0.f, spread = 0.f;
  {
    uint64_t mk = mr;
    while (mk) {
      uint32_t wk[kWalk], wv[kWalk];
      const int n = __popcll(mk);
      next_members(s.K, s.V, mk, lane, wk, wv);
#pragma unroll
      for (int u = 0; u < kWalk; ++u) {
        // absent slots: skip
        if (u < n) {
          const float x0 = bf16_lo(wk[u]) - c0, x1 = bf16_hi(wk[u]) - c1;
          var0 = fmaf(x0, x0, var0);
          var1 = fmaf(x1, x1, var1);
          const float y0 = bf16_lo(wv[u]) - vm0, y1 = bf16_hi(wv[u]) - vm1;
          spread = fmaf(y0, y0, fmaf(y1, y1, spread));
        }
      }
    }
    var0 /= div;
    var1 /= div;
    spread = wave_sum(spread);
  }
  // code[r][kk] = vm_r . bf16(basis)[:, kk]
  {
    float cd[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) cd[kk] = wave_sum(fmaf(vm1, bas1[kk], vm0 * bas0[kk]));
    if (lane == 0) {
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) s.code[r][kk] = cd[kk];
    }
  }
  __syncthreads();
  // detail = bf16(HAAR . code / 4), every wave
  float det[3][8];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const float v = (kHaar[a][0] * s.code[0][kk] + kHaar[a][1] * s.code[1][kk] + kHaar[a][2] * s.code[2][kk] +
                       kHaar[a][3] * s.code[3][kk]) / 4.f;
      det[a][kk] = bf16_to_f32(to_bf16(v));
    }
  }
  const long long pg = (long long)h * p.HP + page;
  if (wave == 0 && lane < 24) p.detail[pg * 24 + lane] = to_bf16(
      (kHaar[lane >> 3][0] * s.code[0][lane & 7] + kHaar[lane >> 3][1] * s.code[1][lane & 7] +
       kHaar[lane >> 3][2] * s.code[2][lane & 7] + kHaar[lane >> 3][3] * s.code[3][lane & 7]) / 4.f);
  // reps, reconstruction error, stats of cluster r
  float e8 = 0.f, e9 = 0.f;
  uint32_t pk_pair;
  {
    float pk[2];
    const float vm[2] = {vm0, vm1};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int d = d0 + j;
      const float mk = 0.25f * (((s.cent[0][d] + s.cent[1][d]) + s.cent[2][d]) + s.cent[3][d]);
      const float km = s.cent[r][d];
      pk[j] = bf16_to_f32(to_bf16(km - mk + s.kmean[d]));
      const float mu = bf16_to_f32(to_bf16(s.vmean[d]));
      float acc = 0.f;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const float c = kHaar[0][r] * det[0][kk] + kHaar[1][r] * det[1][kk] + kHaar[2][r] * det[2][kk];
        acc = fmaf(c, j == 0 ? bas0[kk] : bas1[kk], acc);
      }
      const float x8 = km - pk[j], x9 = vm[j] - (mu + acc);
      e8 = fmaf(x8, x8, e8);
      e9 = fmaf(x9, x9, e9);
    }
    pk_pair = pack_bf16(pk[0], pk[1]);
  }
  reinterpret_cast<uint32_t*>(p.keys)[(pg * 4 + r) * 64 + lane] = pk_pair;
  e8 = wave_sum(e8);
  e9 = wave_sum(e9);
  // [r, 0:8]: mean of the key variance over each 16-dim group (lanes 8g..8g+7)
  float gv = var0 + var1;
  // lanes l ^ 1, l ^ 2 (quad permutations), then l ^ 4 by the half-row mirror
  // (lane l ^ 7, which holds the value of l ^ 4 after the first two steps)
  gv += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(gv), 0xB1, 0xF, 0xF, false));
  gv += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(gv), 0x4E, 0xF, 0xF, false));
  gv += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(gv), 0x141, 0xF, 0xF, false));
  uint16_t* st = p.stats + (pg * 4 + r) * 12;
  if ((lane & 7) == 0) st[lane >> 3] = to_bf16(gv / 16.f);
  // [0, 11] = |mean v - bf16(mean v)|, [1, 11] = max token |v|, [2..3, 11] = 0
  float v11 = 0.f;
  if (r == 0) {
    const float x0 = s.vmean[d0] - bf16_to_f32(to_bf16(s.vmean[d0]));
    const float x1 = s.vmean[d1] - bf16_to_f32(to_bf16(s.vmean[d1]));
    v11 = sqrtf(wave_sum(fmaf(x0, x0, x1 * x1)));
    reinterpret_cast<uint32_t*>(p.mean)[pg * 64 + lane] = pack_bf16(s.vmean[d0], s.vmean[d1]);
  } else if (r == 1) {
    v11 = vmax;
  }
  if (lane == 0) {
    st[8] = to_bf16(sqrtf(e8));
    st[9] = to_bf16(sqrtf(e9));
    st[10] = to_bf16(sqrtf(spread / div));
    st[11] = to_bf16(v11);
  }
}

// The entry points: src_k null reads the pages from the cache itself; a
// non-null `layers` table runs `nlayers` layers in one launch.
int summary_launch(const void* src_k, const void* src_v, long long src_token_stride, long long src_head_stride,
                   const void* k, const void* v, long long kv_token_stride, long long kv_head_stride,
                   const int32_t* init, const void* basis, void* keys, void* mean, void* detail, void* stats,
                   int head_pages, int heads, int first_page, int pages, int iters, hipStream_t stream,
                   const SummaryLayers* layers = nullptr, int nlayers = 1) {
  if (heads <= 0 || pages <= 0 || first_page < 0 || first_page + pages > head_pages || iters < 1 ||
      init == nullptr)
    return (int)hipErrorInvalidValue;
  // the written-through rows move in 16-byte pieces
  if (src_k && ((((uintptr_t)src_k | (uintptr_t)src_v | (uintptr_t)k | (uintptr_t)v) & 15) ||
                ((src_token_stride | src_head_stride | kv_token_stride | kv_head_stride) & 7)))
    return (int)hipErrorInvalidValue;
  SummaryParams p;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.kv_tok = kv_token_stride;
  p.kv_head = kv_head_stride;
  p.src_k = (const uint16_t*)src_k;
  p.src_v = (const uint16_t*)src_v;
  p.src_tok = src_token_stride;
  p.src_head = src_head_stride;
  p.init = init;
  p.basis = (const uint16_t*)basis;
  p.keys = (uint16_t*)keys;
  p.mean = (uint16_t*)mean;
  p.detail = (uint16_t*)detail;
  p.stats = (uint16_t*)stats;
  p.HP = head_pages;
  p.first = first_page;
  p.pages = pages;
  p.iters = iters;
  if (layers)
    hipLaunchKernelGGL((summary_kernel<SummaryLayers>), dim3(pages, heads, nlayers), dim3(256), 0, stream, p,
                       *layers);
  else
    hipLaunchKernelGGL((summary_kernel<OneLayer>), dim3(pages, heads), dim3(256), 0, stream, p, OneLayer{});
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

int ssa_summary(const void* k, const void* v, long long kv_token_stride, long long kv_head_stride,
                const int32_t* init, const void* basis, void* keys, void* mean, void* detail, void* stats,
                int head_pages, int heads, int first_page, int pages, int iters, hipStream_t stream) {
  return summary_launch(nullptr, nullptr, 0, 0, k, v, kv_token_stride, kv_head_stride, init, basis, keys, mean,
                        detail, stats, head_pages, heads, first_page, pages, iters, stream);
}

int ssa_summary_write(const void* src_k, const void* src_v, long long src_token_stride, long long src_head_stride,
                      void* k, void* v, long long kv_token_stride, long long kv_head_stride, const int32_t* init,
                      const void* basis, void* keys, void* mean, void* detail, void* stats, int head_pages,
                      int heads, int first_page, int pages, int iters, hipStream_t stream) {
  if (src_k == nullptr || src_v == nullptr || k == nullptr || v == nullptr) return (int)hipErrorInvalidValue;
  return summary_launch(src_k, src_v, src_token_stride, src_head_stride, k, v, kv_token_stride, kv_head_stride,
                        init, basis, keys, mean, detail, stats, head_pages, heads, first_page, pages, iters, stream);
}

int ssa_summary_layers(int layers, const void* const* k, const void* const* v, long long kv_token_stride,
                       long long kv_head_stride, const int32_t* init, const void* const* basis, void* const* keys,
                       void* const* mean, void* const* detail, void* const* stats, int head_pages, int heads,
                       int first_page, int pages, int iters, hipStream_t stream) {
  if (layers < 1 || layers > kMaxLayers || !k || !v || !basis || !keys || !mean || !detail || !stats)
    return (int)hipErrorInvalidValue;
  SummaryLayers t;
  for (int l = 0; l < layers; ++l) {
    if (!k[l] || !v[l] || !basis[l] || !keys[l] || !mean[l] || !detail[l] || !stats[l])
      return (int)hipErrorInvalidValue;
    t.k[l] = (const uint16_t*)k[l];
    t.v[l] = (const uint16_t*)v[l];
    t.basis[l] = (const uint16_t*)basis[l];
    t.keys[l] = (uint16_t*)keys[l];
    t.mean[l] = (uint16_t*)mean[l];
    t.detail[l] = (uint16_t*)detail[l];
    t.stats[l] = (uint16_t*)stats[l];
  }
  return summary_launch(nullptr, nullptr, 0, 0, k[0], v[0], kv_token_stride, kv_head_stride, init, basis[0], keys[0],
                        mean[0], detail[0], stats[0], head_pages, heads, first_page, pages, iters, stream, &t,
                        layers);
}

}  // extern "C"
