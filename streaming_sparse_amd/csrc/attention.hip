// Fused exact-page attention + summary compensation + softmax-mass merge for
// gfx950 (one kernel), plus the per-rep value prep it reads.
//
// The reference computes, per (query block t, head h) (RV/tuned_attention.py:
// 20-81 and RV/runtime.py:107-133):
//   exact: online softmax over the LUT pages' 64-token K/V       -> (O_e, le)
//   tail : softmax over the reps of the unselected pages, weight of rep r of
//          page p = 2^(q.r/sqrt(D)*log2e); value mean_p + (sum_a HAAR[a,r]
//          detail_pa) . basis^T; log-mass lt = mx + log2(den) + 4      -> (O_t, lt)
//   merge: rho = 1/(1+2^(le-lt)); out = (1-rho) O_e + rho O_t
// which equals ONE softmax over the union of the exact tokens (logit s,
// value v) and the unselected reps (logit z + 4, value mean_p + code_r .
// basis^T).  This kernel runs that union softmax: it walks "units" of 64 keys
// -- first the C exact pages (rows of the resident [L,H,D] cache), then the
// rep tiles of 16 pages x 4 reps whose pages are not all selected -- with a
// single running max/sum and one [64 x 128] accumulator.  Rep values are
// pre-projected by rep_values_kernel (bf16 rows, like the V rows of a page).
//
// Layout per workgroup (2 waves, 64 queries of one head):
//   wave w owns queries 32w..32w+31.  S^T = K . Q^T and O^T = V^T . P^T use
//   v_mfma_f32_32x32x16_bf16 so each lane holds a single query (lane % 32):
//   the softmax state is lane-local.  K is staged in LDS row-major, V is
//   transposed to [dim][key] in LDS with keys permuted (bits 2<->3 swapped) so
//   each lane's 8 P^T values in MFMA k-order are 16 contiguous bytes.
#include "common.h"

using namespace ssa;

namespace {

constexpr int kThreads = 128;
constexpr int kMaxCount = 512;
constexpr int kMaxRepTiles = 32;   // pages <= 512 -> ceil(P/16) <= 32

struct AttnParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* rk;   // rep keys   [H, HP, 4, D]
  const uint16_t* rv;   // rep values [H, HPV, 4, D]
  const int32_t* ids;   // [H, T, C]
  uint16_t* out;
  long long kv_tok, kv_head;   // element strides of a K/V token row and a head
  long long q_tok, q_head;     // element strides of q / out
  int H, T, P, HP, HPV, C;
  float scale_log2;            // log2(e) / sqrt(D)
};

struct Smem {
  alignas(16) uint8_t kbuf[64 * 256];
  alignas(16) uint8_t vt[128 * 128];
  int units[kMaxCount + kMaxRepTiles];
  uint32_t maskw[16];
  int nunits;
};

struct Stage {
  u32x4 k[8];
  u32x4 v[8];
};

__device__ __forceinline__ int k_off(int row, int chunk) { return row * 256 + ((chunk ^ (row & 15)) << 4); }
__device__ __forceinline__ int vt_off(int d, int chunk) {
  return d * 128 + ((chunk ^ ((d & 7) ^ ((d >> 3) & 7))) << 4);
}
// Physical position of key kappa inside a unit's transposed V row.
__device__ __forceinline__ int key_pos(int kappa) {
  return (kappa & ~12) | ((kappa & 4) << 1) | ((kappa & 8) >> 1);
}

__device__ __forceinline__ void load_unit(const AttnParams& p, int e, int h, int tid, Stage& st) {
  const uint16_t* kb;
  const uint16_t* vb;
  long long rs;
  int last = 63;
  if (e >= 0) {
    kb = p.k + (long long)e * 64 * p.kv_tok + (long long)h * p.kv_head;
    vb = p.v + (long long)e * 64 * p.kv_tok + (long long)h * p.kv_head;
    rs = p.kv_tok;
  } else {
    const int rt = -1 - e;
    kb = p.rk + ((long long)h * p.HP * 4 + rt * 64) * kHeadDim;
    vb = p.rv + ((long long)h * p.HPV * 4 + rt * 64) * kHeadDim;
    rs = kHeadDim;
    // rows of pages >= P are re-read from the last valid rep (masked later)
    last = min(63, p.P * 4 - rt * 64 - 1);
  }
  const int c = tid & 15, r0 = tid >> 4;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = min(8 * i + r0, last);
    st.k[i] = ldg16(kb + row * rs + c * 8);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const int row = min(4 * (8 * j + r0) + e4, last);
      st.v[4 * j + e4] = ldg16(vb + row * rs + c * 8);
    }
  }
}

__device__ __forceinline__ void store_unit(Smem& s, int tid, const Stage& st) {
  const int c = tid & 15, r0 = tid >> 4;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 8 * i + r0;
    *reinterpret_cast<u32x4*>(s.kbuf + k_off(row, c)) = st.k[i];
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int g = 8 * j + r0;
    const int pos = key_pos(4 * g);
    const int cc = pos >> 3, half = (pos >> 2) & 1;
    const u32x4 a = st.v[4 * j + 0], b = st.v[4 * j + 1], c2 = st.v[4 * j + 2], d = st.v[4 * j + 3];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int w = i >> 1;
      const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
      const uint32_t lo = __builtin_amdgcn_perm(b[w], a[w], sel);
      const uint32_t hi = __builtin_amdgcn_perm(d[w], c2[w], sel);
      const int dim = 8 * c + i;
      *reinterpret_cast<u32x2*>(s.vt + vt_off(dim, cc) + half * 8) = u32x2{lo, hi};
    }
  }
}

template <bool PRECISE>
__device__ __forceinline__ void compute_unit(const Smem& s, const AttnParams& p, int e, int lane,
                                             const u32x4 (&qop)[8], float& m, float& l, f32x16 (&O)[4]) {
  const int r = lane & 31, hh = lane >> 5;
  f32x16 S0 = {}, S1 = {};
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    const int c = 2 * st + hh;
    const u32x4 a0 = *reinterpret_cast<const u32x4*>(s.kbuf + k_off(r, c));
    const u32x4 a1 = *reinterpret_cast<const u32x4*>(s.kbuf + k_off(32 + r, c));
    S0 = mfma32(a0, qop[st], S0);
    S1 = mfma32(a1, qop[st], S1);
  }
  const float bias = e < 0 ? 4.0f : 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    S0[i] = S0[i] * p.scale_log2 + bias;
    S1[i] = S1[i] * p.scale_log2 + bias;
  }
  if (e < 0) {
    const int rt = -1 - e;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int page0 = 16 * rt + 2 * j + hh, page1 = page0 + 8;
      const bool m0 = page0 >= p.P || ((s.maskw[page0 >> 5] >> (page0 & 31)) & 1u);
      const bool m1 = page1 >= p.P || ((s.maskw[page1 >> 5] >> (page1 & 31)) & 1u);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (m0) S0[4 * j + i] = -INFINITY;
        if (m1) S1[4 * j + i] = -INFINITY;
      }
    }
  }
  float mloc = fmaxf(S0[0], S1[0]);
#pragma unroll
  for (int i = 1; i < 16; ++i) mloc = fmaxf(mloc, fmaxf(S0[i], S1[i]));
  mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
  const float mnew = fmaxf(m, mloc);
  const float muse = mnew == -INFINITY ? 0.0f : mnew;
  const float alpha = __builtin_amdgcn_exp2f(m - muse);
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    S0[i] = __builtin_amdgcn_exp2f(S0[i] - muse);
    S1[i] = __builtin_amdgcn_exp2f(S1[i] - muse);
    sum += S0[i] + S1[i];
  }
  l = l * alpha + sum;
  m = mnew;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) O[dt] *= alpha;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const f32x16& x = (ks >> 1) ? S1 : S0;
    const int o = 8 * (ks & 1);
    const u32x4 pb = {pack_bf16(x[o + 0], x[o + 1]), pack_bf16(x[o + 2], x[o + 3]), pack_bf16(x[o + 4], x[o + 5]),
                      pack_bf16(x[o + 6], x[o + 7])};
    u32x4 pl = {};
    if (PRECISE) {
#pragma unroll
      for (int w = 0; w < 4; ++w)
        pl[w] = pack_bf16(x[o + 2 * w] - bf16_lo(pb[w]), x[o + 2 * w + 1] - bf16_hi(pb[w]));
    }
    const int cc = 2 * ks + hh;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const u32x4 va = *reinterpret_cast<const u32x4*>(s.vt + vt_off(32 * dt + r, cc));
      O[dt] = mfma32(va, pb, O[dt]);
      if (PRECISE) O[dt] = mfma32(va, pl, O[dt]);
    }
  }
}

template <bool PRECISE>
__global__ __launch_bounds__(kThreads, 2) void attn_kernel(AttnParams p) {
  __shared__ Smem s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int work = xcd_remap(blockIdx.x, p.H * p.T);
  const int h = work / p.T, t = work % p.T;
  if (tid < 16) s.maskw[tid] = 0u;
  __syncthreads();
  const int32_t* ids = p.ids + ((long long)h * p.T + t) * p.C;
  for (int i = tid; i < p.C; i += kThreads) {
    const int pg = min(max(ids[i], 0), p.P - 1);
    s.units[i] = pg;
    atomicOr(&s.maskw[pg >> 5], 1u << (pg & 31));
  }
  __syncthreads();
  if (wave == 0) {
    const int R = (p.P + 15) >> 4;
    bool live = false;
    if (lane < R) {
      const int p0 = lane * 16;
      const uint32_t word = (s.maskw[p0 >> 5] >> (p0 & 31)) & 0xffffu;
      const int valid = min(16, p.P - p0);
      const uint32_t vmask = valid >= 16 ? 0xffffu : ((1u << valid) - 1u);
      live = (~word & vmask) != 0u;
    }
    const unsigned long long bal = __ballot(live);
    if (live) s.units[p.C + __popcll(bal & ((1ull << lane) - 1ull))] = -1 - lane;
    if (lane == 0) s.nunits = p.C + __popcll(bal);
  }
  // query operand: lane's query row, dims 16*st + 8*hh + [0,8)
  const int r = lane & 31, hh = lane >> 5;
  const long long qrow = (long long)(t * 64 + wave * 32 + r);
  u32x4 qop[8];
  const uint16_t* qp = p.q + qrow * p.q_tok + (long long)h * p.q_head + 8 * hh;
#pragma unroll
  for (int st = 0; st < 8; ++st) qop[st] = ldg16(qp + 16 * st);
  __syncthreads();
  const int nunits = s.nunits;

  float m = -INFINITY, l = 0.0f;
  f32x16 O[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) O[dt] = f32x16{};
  Stage st;
  load_unit(p, s.units[0], h, tid, st);
  for (int u = 0; u < nunits; ++u) {
    const int e = s.units[u];
    __syncthreads();
    store_unit(s, tid, st);
    __syncthreads();
    if (u + 1 < nunits) load_unit(p, s.units[u + 1], h, tid, st);
    compute_unit<PRECISE>(s, p, e, lane, qop, m, l, O);
  }
  const float lt = l + __shfl_xor(l, 32);
  const float inv = 1.0f / lt;
  uint16_t* op = p.out + qrow * p.q_tok + (long long)h * p.q_head + 4 * hh;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x2 w = {pack_bf16(O[dt][4 * j] * inv, O[dt][4 * j + 1] * inv),
                       pack_bf16(O[dt][4 * j + 2] * inv, O[dt][4 * j + 3] * inv)};
      *reinterpret_cast<u32x2*>(op + 32 * dt + 8 * j) = w;
    }
  }
}

// vrep[h,p,r,:] = bf16(mean[h,p,:] + sum_k (sum_a HAAR[a,r] detail[h,p,a,k]) basis[h,:,k])
__global__ __launch_bounds__(128) void rep_values_kernel(const uint16_t* mean, const uint16_t* detail,
                                                         const uint16_t* basis, uint16_t* vrep, int HP, int HPV) {
  const int pg = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  __shared__ float det[24];
  if (d < 24) det[d] = bf16_to_f32(detail[((long long)h * HP + pg) * 24 + d]);
  __syncthreads();
  const float mu = bf16_to_f32(mean[((long long)h * HP + pg) * kHeadDim + d]);
  float b[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) b[k] = bf16_to_f32(basis[((long long)h * kHeadDim + d) * 8 + k]);
  const float haar[3][4] = {{1, 1, -1, -1}, {1, -1, 1, -1}, {1, -1, -1, 1}};
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    float acc = mu;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float code = haar[0][rr] * det[k] + haar[1][rr] * det[8 + k] + haar[2][rr] * det[16 + k];
      acc += code * b[k];
    }
    vrep[(((long long)h * HPV + pg) * 4 + rr) * kHeadDim + d] = to_bf16(acc);
  }
}

}  // namespace

extern "C" {

int ssa_rep_values(const void* mean, const void* detail, const void* basis, void* rep_values, int heads, int pages,
                   int head_pages, int rep_head_pages, hipStream_t stream) {
  if (heads <= 0 || pages <= 0 || head_pages < pages || rep_head_pages < pages) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(rep_values_kernel, dim3(pages, heads), dim3(128), 0, stream, (const uint16_t*)mean,
                     (const uint16_t*)detail, (const uint16_t*)basis, (uint16_t*)rep_values, head_pages,
                     rep_head_pages);
  return (int)hipGetLastError();
}

int ssa_attention(const void* q, const void* k, const void* v, const void* keys, const void* rep_values,
                  const int32_t* ids, void* out, int n_tokens, int heads, int pages, int head_pages,
                  int rep_head_pages, int count, long long kv_token_stride, long long kv_head_stride, int flags,
                  hipStream_t stream) {
  if (n_tokens <= 0 || n_tokens % 64 || heads <= 0 || pages <= 0 || pages > 512 || count <= 0 ||
      count > kMaxCount || count > pages || head_pages < pages || rep_head_pages < pages)
    return (int)hipErrorInvalidValue;
  AttnParams p;
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.rk = (const uint16_t*)keys;
  p.rv = (const uint16_t*)rep_values;
  p.ids = ids;
  p.out = (uint16_t*)out;
  p.kv_tok = kv_token_stride;
  p.kv_head = kv_head_stride;
  p.q_tok = (long long)heads * kHeadDim;
  p.q_head = kHeadDim;
  p.H = heads;
  p.T = n_tokens / 64;
  p.P = pages;
  p.HP = head_pages;
  p.HPV = rep_head_pages;
  p.C = count;
  p.scale_log2 = kLog2e / sqrtf((float)kHeadDim);
  const dim3 grid(heads * p.T);
  if (flags & 1)
    hipLaunchKernelGGL(attn_kernel<true>, grid, dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(attn_kernel<false>, grid, dim3(kThreads), 0, stream, p);
  return (int)hipGetLastError();
}

}  // extern "C"
