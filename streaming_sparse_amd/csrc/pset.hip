// Full_Pset swap correction for gfx950: page encodings, reader readout with
// FP64 mixture states, and the per-(remove, add) set-gain table with the
// apply step.
//
// Reference (VB = reproduction/vbench_current, VR = local_experiments/
// video_runtime_v1, LE = local_experiments):
//   encode  : f = per-part RMS-normalised [keys|mean|detail|stats] (712);
//             co = bf16(reader MLP(f)) [5,17], A = bf16(phi MLP(f)) [8,4],
//             meanB = mean.B, detailB = detail.(bf16(basis)^T B)
//             (VR/page.py:6-14, VR/runtime.py:89,160-164,
//              LE/e27_adaptive_query/core.py:4-11, coefficients.py:4-8)
//   rows    : per probe m of a query block and page p: lm = LSE_r z - LSE z,
//             rp/beta = co0 + sum_j tanh(u.A_j) co_{j+1} (VR/page.py:17-21),
//             approx = meanB + sum_a c_a detailB_a (VB/graph.py:199-201),
//             then the mixtures H (current selection), target (all exact)
//             and the background of non-candidate pages (VR/scores.py:62-68)
//   scores  : for 16 removes x 32 adds, the FP64 endpoint deltas of the
//             mixture after the swap and 2 E.delta - |delta|^2 averaged over
//             the 16 probes (VR/scores.py:69-91); pools and legality of
//             VB/quota_pool.py:3-46; argmax and the gain > 0 gate of
//             VR/scores.py:102-107; the LUT of VB/graph.py:210.
// The mixture background is kept uncentred (the translation by the
// mass-weighted mean cancels in every delta, VR/reader_reduce.py:55-56).
#include "common.h"

#include <mutex>
#include <type_traits>

using namespace ssa;

namespace {

constexpr int kMaxPages = 512;
constexpr int kAnchors = 24;
constexpr int kCurrent = 72;
constexpr int kFeatures = 712;
constexpr int kMaxHidden = 256;
constexpr int kEncPages = 4;        // pages per encode workgroup (the first-layer weights stream
                                    // through each workgroup once: 4 pages balance that against the FMAs)
static_assert(kEncPages % 4 == 0, "pages go to the four waves in turn");
constexpr int kCoefStride = 128;    // bf16 per page: co[85] | 0 x 11 | A[32]
constexpr int kCoefA = 96;
constexpr int kCand = 48;           // 16 removes + 32 adds
constexpr int kCandVals = 34;       // lm, beta, approx[16], rp[16]
constexpr int kPoolInts = 64;       // 48 candidate pages + 16 legal bit rows

// ------------------------------------------------------------- encoding ----

struct EncodeParams {
  const uint16_t *keys, *mean, *detail, *stats, *basis;
  int HP;
  const float *w1t, *b1, *w2r, *b2r, *w2p, *b2p;
  const double* B;
  uint16_t* coef;
  double *mean_b, *detail_b;
  int EP, first, pages, hidden;
};

// Per-layer tensors of a batched encode (blockIdx.z = layer): the summary
// slab, the basis and the encodings of each layer; the weights are shared.
constexpr int kMaxLayers = 32;
struct EncodeLayers {
  const uint16_t *keys[kMaxLayers], *mean[kMaxLayers], *detail[kMaxLayers], *stats[kMaxLayers],
      *basis[kMaxLayers];
  uint16_t* coef[kMaxLayers];
  double *mean_b[kMaxLayers], *detail_b[kMaxLayers];
};
struct OneLayer {};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <class Layers>
__global__ __launch_bounds__(256) void encode_kernel(EncodeParams p, Layers layers) {
  if constexpr (std::is_same_v<Layers, EncodeLayers>) {
    const int l = blockIdx.z;
    p.keys = layers.keys[l];
    p.mean = layers.mean[l];
    p.detail = layers.detail[l];
    p.stats = layers.stats[l];
    p.basis = layers.basis[l];
    p.coef = layers.coef[l];
    p.mean_b = layers.mean_b[l];
    p.detail_b = layers.detail_b[l];
  }
  __shared__ alignas(16) float f[kFeatures][kEncPages];
  __shared__ alignas(16) float hid[2 * kMaxHidden][kEncPages];
  __shared__ double pb[8][16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.y;
  const int g0 = blockIdx.x * kEncPages;
  const int npg = min(kEncPages, p.pages - g0);

  // features: wave w normalises pages w, w + 4, ...
  for (int j = 0; j < kEncPages / 4; ++j) {
    const int pl = 4 * j + wave;
    if (pl >= npg) break;
    const long long pg = (long long)h * p.HP + p.first + g0 + pl;
    float kv[8];
    const u32x4 k4 = ldg16(p.keys + pg * 512 + lane * 8);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      kv[2 * w] = bf16_lo(k4[w]);
      kv[2 * w + 1] = bf16_hi(k4[w]);
    }
    float ks = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ks += kv[i] * kv[i];
    const uint32_t mw = *reinterpret_cast<const uint32_t*>(p.mean + pg * 128 + lane * 2);
    const float m0 = bf16_lo(mw), m1 = bf16_hi(mw);
    const float dv = lane < 24 ? bf16_to_f32(p.detail[pg * 24 + lane]) : 0.f;
    const float sv = lane < 48 ? bf16_to_f32(p.stats[pg * 48 + lane]) : 0.f;
    const float kd = sqrtf(wave_sum(ks) / 512.f) + 1e-4f;
    const float md = sqrtf(wave_sum(m0 * m0 + m1 * m1) / 128.f) + 1e-4f;
    const float dd = sqrtf(wave_sum(dv * dv) / 24.f) + 1e-4f;
    const float sd = sqrtf(wave_sum(sv * sv) / 48.f) + 1e-4f;
#pragma unroll
    for (int i = 0; i < 8; ++i) f[lane * 8 + i][pl] = kv[i] / kd;
    f[512 + 2 * lane][pl] = m0 / md;
    f[512 + 2 * lane + 1][pl] = m1 / md;
    if (lane < 24) f[640 + lane][pl] = dv / dd;
    if (lane < 48) f[664 + lane][pl] = sv / sd;
  }
  // bf16(basis)^T B for this head
  if (tid < 128) {
    const int k = tid >> 4, e = tid & 15;
    double acc = 0.0;
#pragma unroll 32
    for (int d = 0; d < 128; ++d)
      acc += (double)bf16_to_f32(p.basis[((long long)h * 128 + d) * 8 + k]) * p.B[d * 16 + e];
    pb[k][e] = acc;
  }
  __syncthreads();

  // layer 1 of both MLPs: thread j -> reader hidden j and phi hidden j
  const int H = p.hidden;
  if (tid < H) {
    float ar[kEncPages], ap[kEncPages];
#pragma unroll
    for (int i = 0; i < kEncPages; ++i) ar[i] = ap[i] = 0.f;
    const float* wr = p.w1t + tid;
    const float* wp = p.w1t + H + tid;
    // 32 rows of the weights in flight per thread: the loop streams 1.46 MB
    // of weights through each workgroup and waits on their latency otherwise
#pragma unroll 32
    for (int k = 0; k < kFeatures; ++k) {
      const float a = wr[(long long)k * 2 * H], b = wp[(long long)k * 2 * H];
#pragma unroll
      for (int c = 0; c < kEncPages / 4; ++c) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(&f[k][4 * c]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ar[4 * c + i] = fmaf(x[i], a, ar[4 * c + i]);
          ap[4 * c + i] = fmaf(x[i], b, ap[4 * c + i]);
        }
      }
    }
    const float br = p.b1[tid], bp = p.b1[H + tid];
#pragma unroll
    for (int i = 0; i < kEncPages; ++i) {
      const float xr = ar[i] + br, xp = ap[i] + bp;
      hid[tid][i] = 0.5f * xr * (1.0f + erff(xr * 0.70710678118654752f));
      hid[H + tid][i] = 0.5f * xp * (1.0f + erff(xp * 0.70710678118654752f));
    }
  }
  __syncthreads();

  // layer 2: 85 reader + 32 phi outputs per page, rounded to bf16
  for (int idx = tid; idx < 117 * kEncPages; idx += 256) {
    const int o = idx / kEncPages, pl = idx % kEncPages;
    if (pl >= npg) continue;
    const bool rd = o < 85;
    const float* w = rd ? p.w2r + (long long)o * H : p.w2p + (long long)(o - 85) * H;
    const int off = rd ? 0 : H;
    float acc = 0.f;
    for (int j = 0; j < H; ++j) acc = fmaf(hid[off + j][pl], w[j], acc);
    acc += rd ? p.b2r[o] : p.b2p[o - 85];
    const long long base = ((long long)h * p.EP + p.first + g0 + pl) * kCoefStride;
    p.coef[base + (rd ? o : kCoefA + o - 85)] = to_bf16(acc);
  }
  for (int idx = tid; idx < 11 * kEncPages; idx += 256) {
    const int pl = idx / 11;
    if (pl < npg) p.coef[((long long)h * p.EP + p.first + g0 + pl) * kCoefStride + 85 + idx % 11] = 0;
  }
  // meanB and detailB (fp64)
  for (int idx = tid; idx < kEncPages * 16; idx += 256) {
    const int pl = idx >> 4, e = idx & 15;
    if (pl >= npg) continue;
    const long long pg = (long long)h * p.HP + p.first + g0 + pl;
    double acc = 0.0;
#pragma unroll 32
    for (int d = 0; d < 128; ++d) acc += (double)bf16_to_f32(p.mean[pg * 128 + d]) * p.B[d * 16 + e];
    p.mean_b[((long long)h * p.EP + p.first + g0 + pl) * 16 + e] = acc;
  }
  for (int idx = tid; idx < kEncPages * 48; idx += 256) {
    const int pl = idx / 48, a = (idx / 16) % 3, e = idx & 15;
    if (pl >= npg) continue;
    const long long pg = (long long)h * p.HP + p.first + g0 + pl;
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < 8; ++k) acc += (double)bf16_to_f32(p.detail[pg * 24 + a * 8 + k]) * pb[k][e];
    p.detail_b[(((long long)h * p.EP + p.first + g0 + pl) * 3 + a) * 16 + e] = acc;
  }
}

// ----------------------------------------------------------------- pool ----

struct PsetParams {
  const uint16_t* q;
  long long q_head, q_block, q_row;
  int gathered;
  const uint16_t* rk;
  int HP;
  const uint16_t* coef;
  const double *mean_b, *detail_b;
  int EP;
  const float* wq;
  const float* risk;
  const float* lse;            // [H, T, 16] per-probe LSE over all reps (from the router)
  uint8_t* mask;
  int32_t* ids;
  const int32_t* own;
  const int32_t* heads;
  int HS;
  double *cand, *rows;
  int32_t* pool;
  double* gain;
  int32_t* info;
  double* scores;
  long long* stats;            // [3] executed swaps, corrected rows, non-finite legal scores
  int H, T, P, C;
};

__device__ __forceinline__ int own_page(const PsetParams& p, int h, int t) {
  // clamped into the window like the router's own page (memory safety)
  return min(max(p.own ? p.own[(long long)h * p.T + t] : p.P - p.T + t, 0), p.P - 1);
}

struct PoolSmem {
  float risk[kMaxPages];
  uint8_t sel[kMaxPages];
  uint8_t isadd[kMaxPages];
  unsigned long long key[kMaxPages];
  int cnt[4];                  // movable history, movable current, unselected history, unselected current
  int spare[32];
};

// One workgroup per scoped (head, block): the stratified pools of
// VB/quota_pool.py:3-46 from one descending bitonic sort of 512 keys whose
// group field orders history removes > current removes > history adds >
// current adds; removes rank by ascending risk, adds by descending risk,
// ties -> lower page.  A 72-page window (the anchor frame is the chunk's
// first frame, every other page current: VB/quota_pool.py:21-33) has one
// remove group and one add group: up to 8 movable removes, then the anchor
// pages other than own; the unselected pages by descending risk, then the
// selected pages in page order; the movable removes x the first 16 add
// slots are legal.
__global__ __launch_bounds__(256) void pset_pool_kernel(PsetParams p) {
  __shared__ PoolSmem s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hs = blockIdx.x / p.T, t = blockIdx.x % p.T;
  const int h = p.heads[hs];
  const int P = p.P;
  const long long rowoff = ((long long)h * p.T + t) * P;
  const int own = own_page(p, h, t);
  if (blockIdx.x == 0 && tid < 3) p.stats[tid] = tid == 1 ? (long long)p.HS * p.T : 0ll;
  for (int i = tid; i < kMaxPages; i += 256) {
    s.risk[i] = i < P ? p.risk[rowoff + i] : 0.f;
    s.sel[i] = i < P ? (p.mask[rowoff + i] ? 1 : 0) : 1;
    s.isadd[i] = 0;
  }
  if (tid < 4) s.cnt[tid] = 0;
  __syncthreads();
  const bool first = P == kCurrent;
  for (int pg = tid; pg < kMaxPages; pg += 256) {
    unsigned long long key = 0ull;
    // a 72-page window counts every page in the history groups (4: removes,
    // 2: adds), so its removes and adds each form one contiguous run; its
    // adds range over all pages (an anchor page is selected in every mask
    // the router writes)
    if ((pg >= kAnchors || first) && pg < P) {
      const int cur = first ? 0 : pg >= P - kCurrent;
      const uint32_t ord = orderable(s.risk[pg]);
      int group = 0;
      uint32_t kv = 0;
      if (s.sel[pg] && pg != own && pg >= kAnchors) {
        group = cur ? 3 : 4;
        kv = ~ord;
      } else if (!s.sel[pg]) {
        group = cur ? 1 : 2;
        kv = ord;
      }
      if (group) {
        key = ((unsigned long long)group << 60) | ((unsigned long long)kv << 20) | (unsigned long long)(1023 - pg);
        atomicAdd(&s.cnt[4 - group], 1);
      }
    }
    s.key[pg] = key;
  }
  __syncthreads();
  for (int k = 2; k <= kMaxPages; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int lo = 2 * tid - (tid & (j - 1)), hi = lo + j;
      const bool desc = (lo & k) == 0;
      const unsigned long long a = s.key[lo], c = s.key[hi];
      if ((a < c) == desc) {
        s.key[lo] = c;
        s.key[hi] = a;
      }
      __syncthreads();
    }
  }
  const int nmh = s.cnt[0], nmc = s.cnt[1], nuh = s.cnt[2], nuc = s.cnt[3];
  auto page_at = [&](int i) -> int { return 1023 - (int)(s.key[i] & 1023ull); };
  if (first) {
    // the selected pages in page order fill the add slots past the unselected ones
    if (wave == 0) {
      int cnt = 0;
      for (int base = 0; base < P; base += 64) {
        const int pg = base + lane;
        const bool on = pg < P && s.sel[pg];
        const unsigned long long bal = __ballot(on);
        const int r = cnt + __popcll(bal & ((1ull << lane) - 1ull));
        if (on && r < 32) s.spare[r] = pg;
        cnt += __popcll(bal);
      }
    }
    __syncthreads();
    if (tid < kCand) {
      const int sl = tid, used = min(nmh, 8);
      int page;
      if (sl < 16) {
        // the anchor pages other than own, in page order, stand in past the movable removes
        const int a = sl - used;
        page = sl < used ? page_at(sl) : a + (own < kAnchors && a >= own ? 1 : 0);
      } else {
        const int k = sl - 16;
        page = k < nuh ? page_at(nmh + k) : s.spare[k - nuh];
      }
      int32_t* po = p.pool + ((long long)hs * p.T + t) * kPoolInts;
      po[sl] = page;
      if (sl < 16) po[kCand + sl] = sl < used ? 0xffff : 0;
    }
    return;
  }
  // valid adds, then spare pages (neither selected nor a valid add), ascending
  if (tid < 32) {
    const int q = tid >> 4, k = tid & 15;
    const int n = q ? nuc : nuh;
    if (k < n) s.isadd[page_at(nmh + nmc + (q ? nuh : 0) + k)] = 1;
  }
  __syncthreads();
  if (wave == 0) {
    int cnt = 0;
    for (int base = 0; base < P; base += 64) {
      const int pg = base + lane;
      const bool fr = pg < P && !s.sel[pg] && !s.isadd[pg];
      const unsigned long long bal = __ballot(fr);
      const int r = cnt + __popcll(bal & ((1ull << lane) - 1ull));
      if (fr && r < 32) s.spare[r] = pg;
      cnt += __popcll(bal);
    }
    if (lane < 32 && lane >= cnt) s.spare[lane] = -1;
  }
  __syncthreads();
  if (tid < kCand) {
    const int sl = tid;
    int page;
    bool valid;
    if (sl < 16) {
      const int q = sl >> 3, k = sl & 7;
      valid = k < (q ? nmc : nmh);
      page = valid ? page_at((q ? nmh : 0) + k) : sl;          // anchor stands in (never legal)
    } else {
      const int q = (sl - 16) >> 4, k = (sl - 16) & 15;
      valid = k < (q ? nuc : nuh);
      page = valid ? page_at(nmh + nmc + (q ? nuh : 0) + k) : s.spare[sl - 16];   // spare (never legal)
      if (page < 0) {
        // no spare page left for this slot (the reference's pool would index
        // page P, past the window): an empty candidate -- zero mass (lm =
        // -inf), zero values -- that adds nothing to any sum, while every
        // page outside the pool stays in the background.  The rows kernel
        // writes no endpoint data for it (no page maps to the slot).
        double* c = p.cand + ((((long long)hs * p.T + t) * 16) * kCand + sl) * kCandVals;
        for (int m = 0; m < 16; ++m)
          for (int v = 0; v < kCandVals; ++v) c[(long long)m * kCand * kCandVals + v] = v == 0 ? -INFINITY : 0.0;
      }
    }
    int32_t* po = p.pool + ((long long)hs * p.T + t) * kPoolInts;
    po[sl] = page;
    if (sl < 16) {
      const int q = sl >> 3;
      const int na = q ? nuc : nuh;
      const uint32_t addbits = na >= 16 ? 0xffffu : ((1u << na) - 1u);
      po[kCand + sl] = valid ? (int32_t)(addbits << (16 * q)) : 0;
    }
  }
}

// ----------------------------------------------------------------- rows ----

constexpr int kSplit = 2;          // page ranges per (head, pair of blocks)
constexpr int kRowPart = 52;       // accH[16], accT[16], accB[16], sH, sT, sB, max logs

struct RowsSmem {
  uint8_t sel[2][kMaxPages];
  int8_t slot[2][kMaxPages];       // remove slot (0..15) of a pool page, or -1
  int8_t aslot[2][kMaxPages];      // add slot (16..47), or -1: a 72-page pool may list a page in both
  float u[32][8];
  float L[32];
  alignas(16) float coef[4][8][128];     // per-wave staging of a tile's 8 pages (fp32)
  alignas(16) double md[4][8][64];       // meanB[16] | detailB[48]
  double part[4][32][kRowPart];
};

// One workgroup per (scoped head, pair of blocks, page range): per probe
// and page, the log mass lm = LSE_r z - LSE z, the readout (rp, beta), the
// summary approximation, then partial mixture sums; candidate pages write
// their endpoint data.
__global__ __launch_bounds__(256) void pset_rows_kernel(PsetParams p) {
  __shared__ RowsSmem s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int NP = (p.T + 1) >> 1;
  const int sp = blockIdx.x % kSplit;
  const int pair_id = (blockIdx.x / kSplit) % NP;
  const int hs = blockIdx.x / (kSplit * NP);
  const int t0 = 2 * pair_id;
  const int h = p.heads[hs];
  const int P = p.P;
  const int nrow = min(2, p.T - t0);
  const int ntiles = (P + 7) >> 3;
  const int tile0 = sp * ntiles / kSplit, tile1 = (sp + 1) * ntiles / kSplit;

  for (int i = tid; i < 2 * P; i += 256) {
    const int b = i / P, pg = i % P;
    const int tb = min(t0 + b, p.T - 1);
    s.sel[b][pg] = p.mask[((long long)h * p.T + tb) * P + pg] ? 1 : 0;
    s.slot[b][pg] = -1;
    s.aslot[b][pg] = -1;
  }
  __syncthreads();
  if (tid < 2 * kCand) {
    const int b = tid / kCand, sl = tid % kCand;
    const int tb = min(t0 + b, p.T - 1);
    const int page = p.pool[((long long)hs * p.T + tb) * kPoolInts + sl];
    if (page >= 0 && page < P) (sl < 16 ? s.slot : s.aslot)[b][page] = (int8_t)sl;
  }
  // reader query u = Wq . probe (fp32) and the probe LSE from the router
  {
    const int pr = tid >> 3, i = tid & 7;
    const int tb = min(t0 + (pr >> 4), p.T - 1);
    const long long rr = p.gathered ? (pr & 15) : probe_row(pr & 15);
    const uint16_t* qq = p.q + (long long)h * p.q_head + (long long)tb * p.q_block + rr * p.q_row;
    const f32x4* wr = reinterpret_cast<const f32x4*>(p.wq + i * 128);
    u32x4 qv[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) qv[c] = ldg16(qq + 8 * c);
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const f32x4 w0 = wr[2 * c], w1 = wr[2 * c + 1];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        acc = fmaf(bf16_lo(qv[c][k]), w0[2 * k], acc);
        acc = fmaf(bf16_hi(qv[c][k]), w0[2 * k + 1], acc);
        acc = fmaf(bf16_lo(qv[c][2 + k]), w1[2 * k], acc);
        acc = fmaf(bf16_hi(qv[c][2 + k]), w1[2 * k + 1], acc);
      }
    }
    s.u[pr][i] = acc;
    if (i == 0) s.L[pr] = p.lse[((long long)h * p.T + tb) * 16 + (pr & 15)];
  }
  const int pi = lane & 31, hh = lane >> 5;
  const int blk = pi >> 4, m = pi & 15;
  const int tq = min(t0 + blk, p.T - 1);
  const long long row = p.gathered ? m : probe_row(m);
  const uint16_t* qbase = p.q + (long long)h * p.q_head + (long long)tq * p.q_block + row * p.q_row;
  u32x4 qop[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) qop[st] = ldg16(qbase + 64 * hh + 8 * st);
  __syncthreads();
  float u[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) u[i] = s.u[pi][i];
  const double L = (double)s.L[pi];
  const uint16_t* rkh = p.rk + (long long)h * p.HP * 4 * kHeadDim;
  const float c2 = kLog2e / sqrtf((float)kHeadDim);    // logits in log2 units
  constexpr float kLn2 = 0.69314718055994531f;

  double accH[16], accT[16], accB[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) accH[e] = accT[e] = accB[e] = 0.0;
  double sH = 0.0, sT = 0.0, sB = 0.0, lmax = -INFINITY;
  const long long row_id = ((long long)hs * p.T + tq) * 16 + m;
  float* cw = &s.coef[wave][0][0];
  double* mw = &s.md[wave][0][0];
  // A tile's inputs (the 8 pages' coefficients and meanB | detailB, and its
  // 32 rep keys) are loaded into registers one tile ahead: the loads of the
  // wave's next tile are in flight while this tile's pages are computed.
  u32x4 fa, fb, fm[4], fk[8];
  auto fetch = [&](int tile) {
    const int pl = lane >> 3, c = lane & 7;
    const int page = min(tile * 8 + pl, P - 1);
    const uint16_t* cf = p.coef + ((long long)h * p.EP + page) * kCoefStride + 16 * c;
    const double* src = c < 2 ? p.mean_b + ((long long)h * p.EP + page) * 16 + 8 * c
                               : p.detail_b + ((long long)h * p.EP + page) * 48 + 8 * (c - 2);
    fa = ldg16(cf);
    fb = ldg16(cf + 8);
    const u32x4* s4 = reinterpret_cast<const u32x4*>(src);
#pragma unroll
    for (int k = 0; k < 4; ++k) fm[k] = s4[k];
    const int row = min(tile * 32 + (lane & 31), P * 4 - 1);
    const uint16_t* a = rkh + (long long)row * kHeadDim + 64 * hh;
#pragma unroll
    for (int st = 0; st < 8; ++st) fk[st] = ldg16(a + 8 * st);
  };
  if (tile0 + wave < tile1) fetch(tile0 + wave);
  for (int tile = tile0 + wave; tile < tile1; tile += 4) {
    // stage this tile's 8 pages: coefficients (bf16 -> fp32) and meanB | detailB
    {
      const int pl = lane >> 3, c = lane & 7;
      float* d = cw + pl * 128 + 16 * c;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        d[2 * k] = bf16_lo(fa[k]);
        d[2 * k + 1] = bf16_hi(fa[k]);
        d[8 + 2 * k] = bf16_lo(fb[k]);
        d[8 + 2 * k + 1] = bf16_hi(fb[k]);
      }
      u32x4* md = reinterpret_cast<u32x4*>(mw + pl * 64 + 8 * c);
#pragma unroll
      for (int k = 0; k < 4; ++k) md[k] = fm[k];
    }
    f32x16 S = {};
#pragma unroll
    for (int st = 0; st < 8; ++st) S = mfma32(fk[st], qop[st], S);
    if (tile + 4 < tile1) fetch(tile + 4);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pl = 2 * j + hh;
      const int page = tile * 8 + pl;
      if (page >= P) continue;
      // rep softmax of the page (fp32), page log mass in fp64
      float z[4], w[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = S[4 * j + r] * c2;
      const float zm = fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3]));
      float sw = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        w[r] = __builtin_amdgcn_exp2f(z[r] - zm);
        sw += w[r];
      }
      const double lm = (double)((zm + __log2f(sw)) * kLn2) - L;
      const float isw = 1.0f / sw;
      const float c0 = (w[0] + w[1] - w[2] - w[3]) * isw;
      const float c1 = (w[0] - w[1] + w[2] - w[3]) * isw;
      const float cc2 = (w[0] - w[1] - w[2] + w[3]) * isw;
      // readout: F_j = tanh(u . A_j), val = co_0 + sum_j F_j co_{j+1}
      const float* cf = cw + pl * 128;
      float F[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = fmaf(u[i], cf[kCoefA + 4 * i + jj], acc);
        F[jj] = tanhf(acc);
      }
      float val[17];
#pragma unroll
      for (int k = 0; k < 17; ++k) {
        float acc = 0.f;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc = fmaf(F[jj], cf[(jj + 1) * 17 + k], acc);
        val[k] = cf[k] + acc;
      }
      const double beta = (double)val[16];
      const bool sel = s.sel[blk][page];
      const int sl = s.slot[blk][page], sa = s.aslot[blk][page];
      const bool bg = sl < 0 && sa < 0;      // a background page: in no pool slot
      const double le = lm + beta;
      const double lg = sel ? le : lm;
      lmax = fmax(lmax, lg);
      const double ex = (double)__builtin_amdgcn_exp2f((float)lg * kLog2e);
      const double et = (double)__builtin_amdgcn_exp2f((float)le * kLog2e);
      sH += ex;
      sT += et;
      if (bg) sB += ex;
      const double* md = mw + pl * 64;
      double* cd = (sl >= 0 && blk < nrow) ? p.cand + (row_id * kCand + sl) * kCandVals : nullptr;
      double* ca = (sa >= 0 && blk < nrow) ? p.cand + (row_id * kCand + sa) * kCandVals : nullptr;
      if (cd) {
        cd[0] = lm;
        cd[1] = beta;
      }
      if (ca) {
        ca[0] = lm;
        ca[1] = beta;
      }
      const double d0 = c0, d1 = c1, d2 = cc2;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const double ap = md[e] + (d0 * md[16 + e] + d1 * md[32 + e] + d2 * md[48 + e]);
        const double rp = (double)val[e];
        const double cur = sel ? ap + rp : ap;
        accH[e] += ex * cur;
        accT[e] += et * (ap + rp);
        if (bg) accB[e] += ex * cur;
        if (cd) {
          cd[2 + e] = ap;
          cd[18 + e] = rp;
        }
        if (ca) {
          ca[2 + e] = ap;
          ca[18 + e] = rp;
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  // reduce over the two page halves of a lane pair, then over waves
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    accH[e] += __shfl_xor(accH[e], 32);
    accT[e] += __shfl_xor(accT[e], 32);
    accB[e] += __shfl_xor(accB[e], 32);
  }
  sH += __shfl_xor(sH, 32);
  sT += __shfl_xor(sT, 32);
  sB += __shfl_xor(sB, 32);
  lmax = fmax(lmax, __shfl_xor(lmax, 32));
  if (hh == 0) {
    double* pw = s.part[wave][pi];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      pw[e] = accH[e];
      pw[16 + e] = accT[e];
      pw[32 + e] = accB[e];
    }
    pw[48] = sH;
    pw[49] = sT;
    pw[50] = sB;
    pw[51] = lmax;
  }
  __syncthreads();
  for (int i = tid; i < 32 * kRowPart; i += 256) {
    const int pr = i / kRowPart, e = i % kRowPart;
    if ((pr >> 4) >= nrow) continue;
    double v = e == 51 ? -INFINITY : 0.0;
#pragma unroll
    for (int w = 0; w < 4; ++w) v = e == 51 ? fmax(v, s.part[w][pr][e]) : v + s.part[w][pr][e];
    p.rows[((((long long)hs * p.T + t0 + (pr >> 4)) * 16 + (pr & 15)) * kSplit + sp) * kRowPart + e] = v;
  }
}

// --------------------------------------------------------------- scores ----

struct ScoreSmem {
  alignas(16) double cand[4][kCand][kCandVals];   // per wave: one probe's candidate endpoints
  double V[4][16][kCand];                // endpoint vectors D(c - H) + e^(e-M) rp, [dim][candidate]
  double S[4][kCand];                    // S_r (removes) / T_a (adds), shifted by the row max
  double ex[4][kCand][2];                // e^(lm+beta-M), e^(lm-M) of each candidate
  double Hs[4][48];                      // H[16] | E[16] | ob[16] of the probe
  double sc[4][3];                       // B, shift M, unused
  double acc[4][512];
  alignas(16) double part[4][kSplit * kRowPart];   // the probe's split row partials
  uint32_t legal[16];
  int page[kMaxPages];                   // pool pages, then the compacted selection
  unsigned long long key[kMaxPages];     // LUT keys of the compacted selection
  float risk[kMaxPages];
  uint8_t sel[kMaxPages];
  double best[4];
  int besti[4], bad[4];
};

// One workgroup per scoped (head, block); wave w takes probes w, w+4, ...
// With every log mass shifted by the row max M, e^(-den) of a swap is
// 1/(S_r + T_a) where S_r = B + sum_{k!=r} e^(er_k-M) + e^(lr_r-M) and
// T_a = sum_{k!=a} e^(la_k-M) + e^(ea_a-M) (VR/scores.py:72-73), and each
// endpoint delta of VR/scores.py:81-88 factors into e^(-den) times a
// per-candidate vector, so delta(r,a) = (V_a - V_r) / (S_r + T_a).
__global__ __launch_bounds__(256) void pset_scores_kernel(PsetParams p) {
  __shared__ ScoreSmem s;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int hs = blockIdx.x / p.T, t = blockIdx.x % p.T;
  const int h = p.heads[hs];
  const int P = p.P;
  const long long rowbase = (long long)hs * p.T + t;
  const int32_t* po = p.pool + rowbase * kPoolInts;
  if (tid < kCand) s.page[tid] = po[tid];
  if (tid < 16) s.legal[tid] = (uint32_t)po[kCand + tid];
  for (int i = tid; i < P; i += 256) {
    const long long r = ((long long)h * p.T + t) * P + i;
    s.risk[i] = p.risk[r];
    s.sel[i] = p.mask[r] ? 1 : 0;
  }
  for (int i = lane; i < 512; i += 64) s.acc[w][i] = 0.0;
  // A probe's candidates (48 x 34 doubles = 816 16-byte chunks) and split row
  // partials (kSplit x 52 doubles) are loaded one probe ahead: the loads of
  // probe m + 4 are in flight while probe m is scored.
  constexpr int kChunks = kSplit * kRowPart / 2;
  constexpr int kRowLoads = (kChunks + 63) / 64;
  u32x4 v[13], r[kRowLoads];
  auto load_probe = [&](int m) {
    const u32x4* cd = reinterpret_cast<const u32x4*>(p.cand + (rowbase * 16 + m) * kCand * kCandVals);
#pragma unroll
    for (int k = 0; k < 13; ++k) v[k] = cd[min(lane + 64 * k, 815)];
    const u32x4* rs = reinterpret_cast<const u32x4*>(p.rows + (rowbase * 16 + m) * kSplit * kRowPart);
#pragma unroll
    for (int k = 0; k < kRowLoads; ++k) r[k] = rs[min(64 * k + lane, kChunks - 1)];
  };
  load_probe(w);
  for (int m = w; m < 16; m += 4) {
    // stage the probe's candidates and row state, then request the next probe's
    {
      u32x4* dst = reinterpret_cast<u32x4*>(&s.cand[w][0][0]);
#pragma unroll
      for (int k = 0; k < 13; ++k) {
        const int c = lane + 64 * k;
        if (c < 816) dst[c] = v[k];
      }
      u32x4* pd = reinterpret_cast<u32x4*>(s.part[w]);
#pragma unroll
      for (int k = 0; k < kRowLoads; ++k)
        if (64 * k + lane < kChunks) pd[64 * k + lane] = r[k];
    }
    if (m + 4 < 16) load_probe(m + 4);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < 16) {
      double aH = 0.0, aT = 0.0, aB = 0.0, zH = 0.0, zT = 0.0, zB = 0.0, lx = -INFINITY;
#pragma unroll
      for (int k = 0; k < kSplit; ++k) {
        const double* r = s.part[w] + k * kRowPart;
        aH += r[lane];
        aT += r[16 + lane];
        aB += r[32 + lane];
        zH += r[48];
        zT += r[49];
        zB += r[50];
        lx = fmax(lx, r[51]);
      }
      const double Hv = aH / zH;
      s.Hs[w][lane] = Hv;
      s.Hs[w][16 + lane] = aT / zT - Hv;
      s.Hs[w][32 + lane] = aB / zB;
      if (lane == 0) {
        s.sc[w][0] = zB * exp(-lx);
        s.sc[w][1] = lx;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const double B = s.sc[w][0], M = s.sc[w][1];
    // per candidate: endpoint vector and its share of the swap denominator
    if (lane < kCand) {
      const double* c = s.cand[w][lane];
      const double lmk = c[0], bk = c[1];
      const double EX = exp(lmk + bk - M), LM = exp(lmk - M);
      const double D = fabs(bk) < 0.5 ? LM * expm1(fmin(fmax(bk, -0.5), 0.5)) : EX - LM;
#pragma unroll
      for (int e = 0; e < 16; ++e) s.V[w][e][lane] = D * (c[2 + e] - s.Hs[w][e]) + EX * c[18 + e];
      s.ex[w][lane][0] = EX;
      s.ex[w][lane][1] = LM;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < kCand) {
      // leave-one-out sums over the other candidates of the same group
      double loo = 0.0;
      if (lane < 16) {
        for (int k = 0; k < 16; ++k)
          if (k != lane) loo += s.ex[w][k][0];
        s.S[w][lane] = B + loo + s.ex[w][lane][1];
      } else {
        for (int k = 16; k < kCand; ++k)
          if (k != lane) loo += s.ex[w][k][1];
        s.S[w][lane] = loo + s.ex[w][lane][0];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    uint32_t badmask = 0u;
#pragma unroll 1
    for (int q = 0; q < 8; ++q) {
      const int pr = lane + 64 * q, i = pr >> 5, j = pr & 31;
      const double den = s.S[w][i] + s.S[w][16 + j];
      const double inv = 1.0 / den;
      double ed = 0.0, dd = 0.0;
      bool finite = isfinite(inv);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const double d = (s.V[w][e][16 + j] - s.V[w][e][i]) * inv;
        finite = finite && isfinite(d);
        ed += s.Hs[w][16 + e] * d;
        dd += d * d;
      }
      // the reference's "bad" branch: max logs - den > 80, or a non-finite delta
      if (den < 1.8048513878454153e-35 || !finite) badmask |= 1u << q;
      else s.acc[w][pr] += 2.0 * ed - dd;
    }
    if (__any(badmask != 0u)) {
      // rare: the mixture after the swap rebuilt from the background and every
      // candidate (VR/scores.py:75-79), minus H
#pragma unroll 1
      for (int q = 0; q < 8; ++q) {
        if (!((badmask >> q) & 1u)) continue;
        const int pr = lane + 64 * q, i = pr >> 5, j = pr & 31;
        const double den = s.S[w][i] + s.S[w][16 + j];
        double ed = 0.0, dd = 0.0;
#pragma unroll 1
        for (int e = 0; e < 16; ++e) {
          double nw = B * s.Hs[w][32 + e];
#pragma unroll 1
          for (int k = 0; k < kCand; ++k) {
            const double* c = s.cand[w][k];
            const bool exact = k < 16 ? k != i : k == 16 + j;      // selected after the swap
            nw += exact ? s.ex[w][k][0] * (c[2 + e] + c[18 + e]) : s.ex[w][k][1] * c[2 + e];
          }
          const double d = nw / den - s.Hs[w][e];
          ed += s.Hs[w][16 + e] * d;
          dd += d * d;
        }
        s.acc[w][pr] += 2.0 * ed - dd;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  // legality, argmax (ties -> lowest pair index), finiteness
  double best = -INFINITY;
  int besti = 0x7fffffff;
  int bad = 0;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int flat = tid + 256 * q, i = flat >> 5, j = flat & 31;
    double sc = (((s.acc[0][flat] + s.acc[1][flat]) + s.acc[2][flat]) + s.acc[3][flat]) / 16.0;
    if (!((s.legal[i] >> j) & 1u)) sc = -1e30;
    if (!isfinite(sc)) bad += 1;
    else if (sc > best || (sc == best && flat < besti)) {
      best = sc;
      besti = flat;
    }
    if (p.scores) p.scores[rowbase * 512 + flat] = sc;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const double ob = __shfl_xor(best, o);
    const int oi = __shfl_xor(besti, o);
    bad += __shfl_xor(bad, o);
    if (ob > best || (ob == best && oi < besti)) {
      best = ob;
      besti = oi;
    }
  }
  if (lane == 0) {
    s.best[w] = best;
    s.besti[w] = besti;
    s.bad[w] = bad;
  }
  __syncthreads();
  best = s.best[0];
  besti = s.besti[0];
  bad = s.bad[0];
  for (int k = 1; k < 4; ++k) {
    if (s.best[k] > best || (s.best[k] == best && s.besti[k] < besti)) {
      best = s.best[k];
      besti = s.besti[k];
    }
    bad += s.bad[k];
  }
  const bool exec = bad == 0 && best > 0.0;
  if (tid == 0) {
    p.gain[rowbase] = best;
    p.info[rowbase * 3 + 0] = exec ? 1 : 0;
    p.info[rowbase * 3 + 1] = besti;
    p.info[rowbase * 3 + 2] = bad;
    if (exec) atomicAdd((unsigned long long*)&p.stats[0], 1ull);
    if (bad) atomicAdd((unsigned long long*)&p.stats[2], (unsigned long long)bad);
  }
  if (!exec) return;
  const int rpg = s.page[besti >> 5], apg = s.page[16 + (besti & 31)];
  __syncthreads();
  if (tid == 0) {
    s.sel[rpg] = 0;
    s.sel[apg] = 1;
    const long long base = ((long long)h * p.T + t) * P;
    p.mask[base + rpg] = 0;
    p.mask[base + apg] = 1;
  }
  __syncthreads();
  // LUT of the new selection: own first, then the other selected pages by
  // descending risk, ties -> lower page (compact list, then rank within it)
  if (!p.ids) return;
  const int own = own_page(p, h, t);
  int32_t* ids = p.ids + ((long long)h * p.T + t) * p.C;
  if (w == 0) {
    int cnt = 0;
    for (int base = 0; base < P; base += 64) {
      const int pg = base + lane;
      const bool on = pg < P && s.sel[pg] && pg != own;
      const unsigned long long bal = __ballot(on);
      if (on) s.page[cnt + __popcll(bal & ((1ull << lane) - 1ull))] = pg;   // pool pages no longer needed
      cnt += __popcll(bal);
    }
    if (lane == 0) s.besti[0] = cnt;
  }
  __syncthreads();
  const int nsel = s.besti[0];
  // key (orderable risk, 1023 - page): a higher key ranks first, ties go to
  // the lower page; a page's slot is the count of listed keys above its own
  for (int i = tid; i < nsel; i += 256) {
    const int x = s.page[i];
    s.key[i] = ((unsigned long long)orderable(s.risk[x]) << 32) | (uint32_t)(1023 - x);
  }
  __syncthreads();
  if (tid == 0) ids[0] = own;
  for (int i = tid; i < nsel; i += 256) {
    const unsigned long long kx = s.key[i];
    int rank = 0;
    for (int k = 0; k < nsel; ++k) rank += s.key[k] > kx;
    if (1 + rank < p.C) ids[1 + rank] = s.page[i];
  }
  // a selection shorter than the table (quotas clamped to their partitions)
  // leaves -1 padding, as the router writes it
  for (int i = 1 + nsel + tid; i < p.C; i += 256) ids[i] = -1;
}

// Both entry points: a non-null `layers` table runs `nlayers` layers in one
// launch (entry 0's tensors are also the single-layer arguments).
int encode_launch(const EncodeLayers* layers, int nlayers, const void* keys, const void* mean, const void* detail,
                  const void* stats, int head_pages, const void* basis, const float* w1t, const float* b1,
                  const float* w2_reader, const float* b2_reader, const float* w2_phi, const float* b2_phi,
                  const double* B, void* coef, double* mean_b, double* detail_b, int enc_pages, int heads,
                  int first_page, int pages, int hidden, hipStream_t stream) {
  if (heads <= 0 || pages <= 0 || first_page < 0 || first_page + pages > head_pages ||
      first_page + pages > enc_pages || hidden <= 0 || hidden > kMaxHidden)
    return (int)hipErrorInvalidValue;
  EncodeParams p;
  p.keys = (const uint16_t*)keys;
  p.mean = (const uint16_t*)mean;
  p.detail = (const uint16_t*)detail;
  p.stats = (const uint16_t*)stats;
  p.basis = (const uint16_t*)basis;
  p.HP = head_pages;
  p.w1t = w1t;
  p.b1 = b1;
  p.w2r = w2_reader;
  p.b2r = b2_reader;
  p.w2p = w2_phi;
  p.b2p = b2_phi;
  p.B = B;
  p.coef = (uint16_t*)coef;
  p.mean_b = mean_b;
  p.detail_b = detail_b;
  p.EP = enc_pages;
  p.first = first_page;
  p.pages = pages;
  p.hidden = hidden;
  const dim3 grid((pages + kEncPages - 1) / kEncPages, heads, nlayers);
  if (layers)
    hipLaunchKernelGGL((encode_kernel<EncodeLayers>), grid, dim3(256), 0, stream, p, *layers);
  else
    hipLaunchKernelGGL((encode_kernel<OneLayer>), grid, dim3(256), 0, stream, p, OneLayer{});
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

int ssa_encode(const void* keys, const void* mean, const void* detail, const void* stats, int head_pages,
               const void* basis, const float* w1t, const float* b1, const float* w2_reader, const float* b2_reader,
               const float* w2_phi, const float* b2_phi, const double* B, void* coef, double* mean_b,
               double* detail_b, int enc_pages, int heads, int first_page, int pages, int hidden,
               hipStream_t stream) {
  return encode_launch(nullptr, 1, keys, mean, detail, stats, head_pages, basis, w1t, b1, w2_reader, b2_reader,
                       w2_phi, b2_phi, B, coef, mean_b, detail_b, enc_pages, heads, first_page, pages, hidden, stream);
}

int ssa_encode_layers(int layers, const void* const* keys, const void* const* mean, const void* const* detail,
                      const void* const* stats, int head_pages, const void* const* basis, const float* w1t,
                      const float* b1, const float* w2_reader, const float* b2_reader, const float* w2_phi,
                      const float* b2_phi, const double* B, void* const* coef, double* const* mean_b,
                      double* const* detail_b, int enc_pages, int heads, int first_page, int pages, int hidden,
                      hipStream_t stream) {
  if (layers < 1 || layers > kMaxLayers || !keys || !mean || !detail || !stats || !basis || !coef || !mean_b ||
      !detail_b)
    return (int)hipErrorInvalidValue;
  EncodeLayers t;
  for (int l = 0; l < layers; ++l) {
    if (!keys[l] || !mean[l] || !detail[l] || !stats[l] || !basis[l] || !coef[l] || !mean_b[l] || !detail_b[l])
      return (int)hipErrorInvalidValue;
    t.keys[l] = (const uint16_t*)keys[l];
    t.mean[l] = (const uint16_t*)mean[l];
    t.detail[l] = (const uint16_t*)detail[l];
    t.stats[l] = (const uint16_t*)stats[l];
    t.basis[l] = (const uint16_t*)basis[l];
    t.coef[l] = (uint16_t*)coef[l];
    t.mean_b[l] = mean_b[l];
    t.detail_b[l] = detail_b[l];
  }
  return encode_launch(&t, layers, keys[0], mean[0], detail[0], stats[0], head_pages, basis[0], w1t, b1, w2_reader,
                       b2_reader, w2_phi, b2_phi, B, coef[0], mean_b[0], detail_b[0], enc_pages, heads, first_page,
                       pages, hidden, stream);
}

}  // extern "C"

namespace {

// The three launches of one Full_Pset correction, after argument checks.
int pset_launch(const void* q, long long q_head_stride, long long q_block_stride, long long q_row_stride,
                int gathered, const void* keys, int head_pages, const void* coef, const double* mean_b,
                const double* detail_b, int enc_pages, const float* wq, const float* risk, const float* probe_lse,
                uint8_t* mask, int32_t* ids, const int32_t* own, const int32_t* heads, int n_heads, double* cand,
                double* rows, int32_t* pool, double* gain, int32_t* info, double* scores, long long* stats,
                int total_heads, int blocks, int pages, int count, hipStream_t stream) {
  // a 72-page window (the first chunk) or a window beyond the anchor frame
  // and the current chunk; any table size (an add slot past the spare pages
  // is an empty candidate)
  const bool first = pages == kCurrent;
  if (n_heads <= 0 || n_heads > total_heads || blocks <= 0 || pages > kMaxPages ||
      (!first && pages <= kAnchors + kCurrent) || head_pages < pages ||
      enc_pages < pages || count < (first ? kAnchors : 1) || count > pages ||
      heads == nullptr || probe_lse == nullptr || cand == nullptr || rows == nullptr || pool == nullptr ||
      gain == nullptr || info == nullptr || stats == nullptr)
    return (int)hipErrorInvalidValue;
  PsetParams p;
  p.q = (const uint16_t*)q;
  p.q_head = q_head_stride;
  p.q_block = q_block_stride;
  p.q_row = q_row_stride;
  p.gathered = gathered;
  p.rk = (const uint16_t*)keys;
  p.HP = head_pages;
  p.coef = (const uint16_t*)coef;
  p.mean_b = mean_b;
  p.detail_b = detail_b;
  p.EP = enc_pages;
  p.wq = wq;
  p.risk = risk;
  p.lse = probe_lse;
  p.mask = mask;
  p.ids = ids;
  p.own = own;
  p.heads = heads;
  p.HS = n_heads;
  p.cand = cand;
  p.rows = rows;
  p.pool = pool;
  p.gain = gain;
  p.info = info;
  p.scores = scores;
  p.stats = stats;
  p.H = total_heads;
  p.T = blocks;
  p.P = pages;
  p.C = count;
  const int np = (blocks + 1) / 2;
  hipLaunchKernelGGL(pset_pool_kernel, dim3(n_heads * blocks), dim3(256), 0, stream, p);
  hipLaunchKernelGGL(pset_rows_kernel, dim3(n_heads * np * kSplit), dim3(256), 0, stream, p);
  hipLaunchKernelGGL(pset_scores_kernel, dim3(n_heads * blocks), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

// Scratch of the allocation-free entry point: for at most kScratchRows
// scoped (head, query block) rows, the candidate endpoint data
// [rows,16,48,34] fp64, then the split row partials [rows,16,2,52] fp64, then
// the pools [rows,64] int32, each region at a fixed offset (48.05 MB in all).
// Every entry a call reads is written earlier in the same call (the pool
// kernel writes all 48 slots of each row, the rows kernel the candidates'
// endpoint data and every row partial), so nothing in it must start at zero.
constexpr int kScratchRows = 216;   // 3 heads x 72 query blocks
constexpr size_t kCandRowBytes = (size_t)16 * kCand * kCandVals * sizeof(double);
constexpr size_t kRowsRowBytes = (size_t)16 * kSplit * kRowPart * sizeof(double);
constexpr size_t kPoolRowBytes = (size_t)kPoolInts * sizeof(int32_t);
constexpr size_t kScratchRowsOff = kScratchRows * kCandRowBytes;
constexpr size_t kScratchPoolOff = kScratchRowsOff + kScratchRows * kRowsRowBytes;
constexpr size_t kScratchBytes = kScratchPoolOff + kScratchRows * kPoolRowBytes;
static_assert(kCandRowBytes % 256 == 0 && kRowsRowBytes % 256 == 0, "regions stay 256-byte aligned");

}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

// Device address of `scratch` on each device, looked up once per device with
// that device current (the array's name in host code is only a stand-in).
constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
uint8_t* scratch_ptr[kMaxDevices] = {};

int device_scratch(uint8_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    scratch_ptr[dev] = (uint8_t*)ptr;
  }
  *out = scratch_ptr[dev];
  return (int)hipSuccess;
}

}  // namespace

extern "C" {

int ssa_pset(const void* q, long long q_head_stride, long long q_block_stride, long long q_row_stride,
             int gathered, const void* keys, int head_pages, const void* coef, const double* mean_b,
             const double* detail_b, int enc_pages, const float* wq, const float* risk, const float* probe_lse,
             uint8_t* mask, int32_t* ids, const int32_t* own, const int32_t* heads, int n_heads, double* cand,
             double* rows, int32_t* pool, double* gain, int32_t* info, double* scores, long long* stats,
             int total_heads, int blocks, int pages, int count, hipStream_t stream) {
  return pset_launch(q, q_head_stride, q_block_stride, q_row_stride, gathered, keys, head_pages, coef, mean_b,
                     detail_b, enc_pages, wq, risk, probe_lse, mask, ids, own, heads, n_heads, cand, rows, pool, gain,
                     info, scores, stats, total_heads, blocks, pages, count, stream);
}

int ssa_pset_noalloc(const void* q, long long q_head_stride, long long q_block_stride, long long q_row_stride,
                     int gathered, const void* keys, int head_pages, const void* coef, const double* mean_b,
                     const double* detail_b, int enc_pages, const float* wq, const float* risk,
                     const float* probe_lse, uint8_t* mask, int32_t* ids, const int32_t* own, const int32_t* heads,
                     int n_heads, double* gain, int32_t* info, double* scores, long long* stats, int total_heads,
                     int blocks, int pages, int count, hipStream_t stream) {
  if (n_heads <= 0 || blocks <= 0 || (long long)n_heads * blocks > kScratchRows) return (int)hipErrorInvalidValue;
  uint8_t* base = nullptr;
  const int e = device_scratch(&base);
  if (e != (int)hipSuccess) return e;
  return pset_launch(q, q_head_stride, q_block_stride, q_row_stride, gathered, keys, head_pages, coef, mean_b,
                     detail_b, enc_pages, wq, risk, probe_lse, mask, ids, own, heads, n_heads, (double*)base,
                     (double*)(base + kScratchRowsOff), (int32_t*)(base + kScratchPoolOff), gain, info, scores,
                     stats, total_heads, blocks, pages, count, stream);
}

}  // extern "C"
