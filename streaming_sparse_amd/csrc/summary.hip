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
// One workgroup (256 threads) per (page, head); the page's K and V are
// staged in LDS as fp32 rows padded to 129 floats (conflict-free column
// walks).  Distances and the assignment use thread (token, cluster);
// centroid updates use thread (cluster, dim).
#include "common.h"

using namespace ssa;

namespace {

constexpr int kStride = 129;
constexpr float kHaar[3][4] = {{1, 1, -1, -1}, {1, -1, 1, -1}, {1, -1, -1, 1}};

struct SummaryParams {
  const uint16_t *k, *v;
  long long kv_tok, kv_head;
  const int32_t* init;          // [H, pages, 4] initial tokens
  const uint16_t* basis;        // [H, 128, 8]
  uint16_t *keys, *mean, *detail, *stats;
  int HP, first, pages, iters;
};

struct SumSmem {
  float K[64 * kStride];
  float V[64 * kStride];
  float cent[4][128];
  float vm[4][128];
  float kmean[128], vmean[128];
  float bas[128][8];
  float code[4][8];
  float det[3][8];
  float red[4][128];            // scratch per-cluster partials
  int assign[64];
  int cnt[4];
  float vnorm[64];
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__global__ __launch_bounds__(256) void summary_kernel(SummaryParams p) {
  __shared__ SumSmem s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int pl = blockIdx.x, h = blockIdx.y;
  const int page = p.first + pl;
  const long long base = (long long)page * 64 * p.kv_tok + (long long)h * p.kv_head;
  // stage K and V (fp32)
  for (int i = tid; i < 64 * 16; i += 256) {
    const int t = i >> 4, c = i & 15;
    const u32x4 a = ldg16(p.k + base + t * p.kv_tok + 8 * c);
    const u32x4 b = ldg16(p.v + base + t * p.kv_tok + 8 * c);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      s.K[t * kStride + 8 * c + 2 * w] = bf16_lo(a[w]);
      s.K[t * kStride + 8 * c + 2 * w + 1] = bf16_hi(a[w]);
      s.V[t * kStride + 8 * c + 2 * w] = bf16_lo(b[w]);
      s.V[t * kStride + 8 * c + 2 * w + 1] = bf16_hi(b[w]);
    }
  }
  for (int i = tid; i < 128 * 8; i += 256) s.bas[i >> 3][i & 7] = bf16_to_f32(p.basis[(long long)h * 1024 + i]);
  __syncthreads();
  const int32_t* ini = p.init + ((long long)h * p.pages + pl) * 4;
  for (int i = tid; i < 512; i += 256) {
    const int r = i >> 7, d = i & 127;
    s.cent[r][d] = s.K[ini[r] * kStride + d];
  }
  if (tid < 128) {
    float ks = 0.f, vs = 0.f;
    for (int t = 0; t < 64; ++t) {
      ks += s.K[t * kStride + tid];
      vs += s.V[t * kStride + tid];
    }
    s.kmean[tid] = ks / 64.f;
    s.vmean[tid] = vs / 64.f;
  }
  if (tid < 64) {
    float n = 0.f;
    for (int d = 0; d < 128; ++d) n = fmaf(s.V[tid * kStride + d], s.V[tid * kStride + d], n);
    s.vnorm[tid] = sqrtf(n);
  }
  __syncthreads();

  // Lloyd iterations: assign each token to its nearest centroid (ties ->
  // lower cluster), then move every non-empty centroid to its cluster mean
  for (int it = 0; it < p.iters; ++it) {
    {
      const int t = tid >> 2, r = tid & 3;
      float dist = 0.f;
      for (int d = 0; d < 128; ++d) {
        const float x = s.K[t * kStride + d] - s.cent[r][d];
        dist = fmaf(x, x, dist);
      }
      // argmin over the 4 lanes of this token (lanes 4t..4t+3 of the wave)
      float best = dist;
      int bi = r;
#pragma unroll
      for (int o = 1; o < 4; o <<= 1) {
        const float ob = __shfl_xor(best, o);
        const int oi = __shfl_xor(bi, o);
        if (ob < best || (ob == best && oi < bi)) {
          best = ob;
          bi = oi;
        }
      }
      if (r == 0) s.assign[t] = bi;
    }
    __syncthreads();
    for (int i = tid; i < 512; i += 256) {
      const int r = i >> 7, d = i & 127;
      float sum = 0.f;
      int c = 0;
      for (int t = 0; t < 64; ++t) {
        if (s.assign[t] == r) {
          sum += s.K[t * kStride + d];
          ++c;
        }
      }
      if (c > 0) s.cent[r][d] = sum / (float)c;
      if (d == 0) s.cnt[r] = c;
    }
    __syncthreads();
  }

  // cluster V means (empty cluster -> page V mean) and the key variance
  for (int i = tid; i < 512; i += 256) {
    const int r = i >> 7, d = i & 127;
    const int c = s.cnt[r];
    float sum = 0.f, var = 0.f;
    for (int t = 0; t < 64; ++t) {
      if (s.assign[t] == r) {
        sum += s.V[t * kStride + d];
        const float x = s.K[t * kStride + d] - s.cent[r][d];
        var = fmaf(x, x, var);
      }
    }
    s.vm[r][d] = c > 0 ? sum / (float)c : s.vmean[d];
    s.red[r][d] = var / (float)max(c, 1);
  }
  __syncthreads();
  // code = vm . bf16(basis), detail = bf16(HAAR . code / 4)
  if (tid < 32) {
    const int r = tid >> 3, kk = tid & 7;
    float acc = 0.f;
    for (int d = 0; d < 128; ++d) acc = fmaf(s.vm[r][d], s.bas[d][kk], acc);
    s.code[r][kk] = acc;
  }
  __syncthreads();
  const long long pg = (long long)h * p.HP + page;
  if (tid < 24) {
    const int a = tid >> 3, kk = tid & 7;
    const float v = (kHaar[a][0] * s.code[0][kk] + kHaar[a][1] * s.code[1][kk] + kHaar[a][2] * s.code[2][kk] +
                     kHaar[a][3] * s.code[3][kk]) / 4.f;
    const uint16_t b = to_bf16(v);
    s.det[a][kk] = bf16_to_f32(b);
    p.detail[pg * 24 + tid] = b;
  }
  __syncthreads();
  // wave r handles cluster r: reps, reconstruction error, spreads, stats
  {
    const int r = wave;
    float kmm[2], pk[2], rec[2];
    float e8 = 0.f, e9 = 0.f, gvar[2];
    for (int j = 0; j < 2; ++j) {
      const int d = lane + 64 * j;
      const float mk = 0.25f * (((s.cent[0][d] + s.cent[1][d]) + s.cent[2][d]) + s.cent[3][d]);
      kmm[j] = s.cent[r][d];
      const uint16_t b = to_bf16(s.cent[r][d] - mk + s.kmean[d]);
      pk[j] = bf16_to_f32(b);
      p.keys[(pg * 4 + r) * 128 + d] = b;
      const float mu = bf16_to_f32(to_bf16(s.vmean[d]));
      float acc = 0.f;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const float c = kHaar[0][r] * s.det[0][kk] + kHaar[1][r] * s.det[1][kk] + kHaar[2][r] * s.det[2][kk];
        acc = fmaf(c, s.bas[d][kk], acc);
      }
      rec[j] = mu + acc;
      const float x8 = kmm[j] - pk[j], x9 = s.vm[r][d] - rec[j];
      e8 = fmaf(x8, x8, e8);
      e9 = fmaf(x9, x9, e9);
      gvar[j] = s.red[r][d];
    }
    e8 = wave_sum(e8);
    e9 = wave_sum(e9);
    // [r, 0:8]: mean of the variance over each 16-dim group (lanes 16g..16g+15
    // hold dims 16g.. for g < 4, and 64 + 16g.. for g >= 4)
    float g0 = gvar[0], g1 = gvar[1];
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) {
      g0 += __shfl_xor(g0, o);
      g1 += __shfl_xor(g1, o);
    }
    // V spread: sqrt(sum_t in cluster |v_t - vm_r|^2 / max(n, 1))
    float spread = 0.f;
    for (int t = 0; t < 64; ++t) {
      if (s.assign[t] != r) continue;
      const float x0 = s.V[t * kStride + lane] - s.vm[r][lane];
      const float x1 = s.V[t * kStride + 64 + lane] - s.vm[r][64 + lane];
      spread = fmaf(x0, x0, fmaf(x1, x1, spread));
    }
    spread = wave_sum(spread);
    uint16_t* st = p.stats + (pg * 4 + r) * 12;
    if ((lane & 15) == 0) {
      st[lane >> 4] = to_bf16(g0 / 16.f);
      st[4 + (lane >> 4)] = to_bf16(g1 / 16.f);
    }
    if (lane == 0) {
      st[8] = to_bf16(sqrtf(e8));
      st[9] = to_bf16(sqrtf(e9));
      st[10] = to_bf16(sqrtf(spread / (float)max(s.cnt[r], 1)));
    }
    if (lane == 1) {
      float v11 = 0.f;
      if (r == 0) {
        float e = 0.f;
        for (int d = 0; d < 128; ++d) {
          const float x = s.vmean[d] - bf16_to_f32(to_bf16(s.vmean[d]));
          e = fmaf(x, x, e);
        }
        v11 = sqrtf(e);
      } else if (r == 1) {
        for (int t = 0; t < 64; ++t) v11 = fmaxf(v11, s.vnorm[t]);
      }
      st[11] = to_bf16(v11);
    }
  }
  if (tid < 128) p.mean[pg * 128 + tid] = to_bf16(s.vmean[tid]);
}

}  // namespace

extern "C" {

int ssa_summary(const void* k, const void* v, long long kv_token_stride, long long kv_head_stride,
                const int32_t* init, const void* basis, void* keys, void* mean, void* detail, void* stats,
                int head_pages, int heads, int first_page, int pages, int iters, hipStream_t stream) {
  if (heads <= 0 || pages <= 0 || first_page < 0 || first_page + pages > head_pages || iters < 1 ||
      init == nullptr)
    return (int)hipErrorInvalidValue;
  SummaryParams p;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.kv_tok = kv_token_stride;
  p.kv_head = kv_head_stride;
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
  hipLaunchKernelGGL(summary_kernel, dim3(pages, heads), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

}  // extern "C"
