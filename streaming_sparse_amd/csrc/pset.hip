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

using namespace ssa;

namespace {

constexpr int kMaxPages = 512;
constexpr int kAnchors = 24;
constexpr int kCurrent = 72;
constexpr int kFeatures = 712;
constexpr int kMaxHidden = 256;
constexpr int kEncPages = 8;        // pages per encode workgroup
constexpr int kCoefStride = 128;    // bf16 per page: co[85] | 0 x 11 | A[32]
constexpr int kCoefA = 96;
constexpr int kCand = 48;           // 16 removes + 32 adds
constexpr int kCandVals = 34;       // lm, beta, approx[16], rp[16]
constexpr int kRowVals = 52;        // H[16], E[16], ob[16], lb, logmax, -, -
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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__global__ __launch_bounds__(256) void encode_kernel(EncodeParams p) {
  __shared__ alignas(16) float f[kFeatures][kEncPages];
  __shared__ alignas(16) float hid[2 * kMaxHidden][kEncPages];
  __shared__ double pb[8][16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.y;
  const int g0 = blockIdx.x * kEncPages;
  const int npg = min(kEncPages, p.pages - g0);

  // features: each wave normalises two pages
  for (int j = 0; j < 2; ++j) {
    const int pl = 2 * wave + j;
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
    for (int k = 0; k < kFeatures; ++k) {
      const float a = wr[(long long)k * 2 * H], b = wp[(long long)k * 2 * H];
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(&f[k][0]);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(&f[k][4]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ar[i] = fmaf(x0[i], a, ar[i]);
        ar[4 + i] = fmaf(x1[i], a, ar[4 + i]);
        ap[i] = fmaf(x0[i], b, ap[i]);
        ap[4 + i] = fmaf(x1[i], b, ap[4 + i]);
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

// ----------------------------------------------------------------- rows ----

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
  int H, T, P, C;
};

__constant__ int kProbeOffsets[16] = {0, 4, 8, 13, 17, 21, 25, 29, 34, 38, 42, 46, 50, 55, 59, 63};

struct RowsSmem {
  float risk[2][kMaxPages];
  uint8_t sel[2][kMaxPages];
  uint8_t isadd[2][kMaxPages];
  int8_t slot[2][kMaxPages];
  int rslot[2][16];
  int aslot[2][32];
  int spare[2][32];
  int cnt[2][4];                       // movable hist/cur, unselected hist/cur
  float u[32][8];
  double lse[4][32][2];
  double part[4][32][kRowVals];
};

__device__ __forceinline__ int own_page(const PsetParams& p, int h, int t) {
  return p.own ? p.own[(long long)h * p.T + t] : p.P - p.T + t;
}

__device__ __forceinline__ void rep_tile(const uint16_t* rkh, int tile, int P, int lane, const u32x4 (&qop)[8],
                                         f32x16& S) {
  const int hh = lane >> 5;
  const int row = min(tile * 32 + (lane & 31), P * 4 - 1);
  const uint16_t* a = rkh + (long long)row * kHeadDim + 64 * hh;
  u32x4 av[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) av[st] = ldg16(a + 8 * st);
  S = f32x16{};
#pragma unroll
  for (int st = 0; st < 8; ++st) S = mfma32(av[st], qop[st], S);
}

// log-sum-exp of the 4 rep logits of a page (fp64) and the softmax weights
__device__ __forceinline__ double page_lse(const float (&z)[4], double (&w)[4]) {
  const double zm = (double)fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3]));
  double s = 0.0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    w[r] = exp((double)z[r] - zm);
    s += w[r];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) w[r] /= s;
  return zm + log(s);
}

__global__ __launch_bounds__(256) void pset_rows_kernel(PsetParams p) {
  __shared__ RowsSmem s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int NP = (p.T + 1) >> 1;
  const int hs = blockIdx.x / NP, t0 = 2 * (blockIdx.x % NP);
  const int h = p.heads[hs];
  const int P = p.P;
  const int nrow = min(2, p.T - t0);

  // ---- rows of risk / selection, pools (VB/quota_pool.py:3-46)
  for (int i = tid; i < 2 * P; i += 256) {
    const int b = i / P, pg = i % P;
    const int tb = min(t0 + b, p.T - 1);
    const long long r = ((long long)h * p.T + tb) * P + pg;
    s.risk[b][pg] = p.risk[r];
    s.sel[b][pg] = p.mask[r] ? 1 : 0;
    s.isadd[b][pg] = 0;
    s.slot[b][pg] = -1;
  }
  if (tid < 2 * 16) s.rslot[tid >> 4][tid & 15] = -1;
  if (tid < 2 * 32) s.aslot[tid >> 5][tid & 31] = -1;
  if (tid < 8) s.cnt[tid >> 2][tid & 3] = 0;
  __syncthreads();
  int own[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) own[b] = own_page(p, h, min(t0 + b, p.T - 1));
  for (int i = tid; i < 2 * P; i += 256) {
    const int b = i / P, pg = i % P;
    if (pg < kAnchors) continue;
    const int part = pg >= P - kCurrent ? 1 : 0;
    const int lo = part ? P - kCurrent : kAnchors, hi = part ? P : P - kCurrent;
    const bool sel = s.sel[b][pg];
    const uint32_t key = orderable(s.risk[b][pg]);
    if (sel && pg != own[b]) {
      // removes: ascending risk, ties -> lower page
      int rank = 0;
      for (int y = lo; y < hi; ++y) {
        if (!s.sel[b][y] || y == own[b]) continue;
        const uint32_t ky = orderable(s.risk[b][y]);
        rank += (ky < key) || (ky == key && y < pg);
      }
      if (rank < 8) s.rslot[b][part * 8 + rank] = pg;
      atomicAdd(&s.cnt[b][part], 1);
    } else if (!sel) {
      // adds: descending risk, ties -> lower page
      int rank = 0;
      for (int y = lo; y < hi; ++y) {
        if (s.sel[b][y]) continue;
        const uint32_t ky = orderable(s.risk[b][y]);
        rank += (ky > key) || (ky == key && y < pg);
      }
      if (rank < 16) {
        s.aslot[b][part * 16 + rank] = pg;
        s.isadd[b][pg] = 1;
      }
      atomicAdd(&s.cnt[b][2 + part], 1);
    }
  }
  __syncthreads();
  if (wave < 2) {
    // spare pages: neither selected nor a valid add, ascending index
    const int b = wave;
    int cnt = 0;
    for (int base = 0; base < P; base += 64) {
      const int pg = base + lane;
      const bool fr = pg < P && !s.sel[b][pg] && !s.isadd[b][pg];
      const unsigned long long bal = __ballot(fr);
      const int r = cnt + __popcll(bal & ((1ull << lane) - 1ull));
      if (fr && r < 32) s.spare[b][r] = pg;
      cnt += __popcll(bal);
    }
    if (lane < 32 && lane >= cnt) s.spare[b][lane] = -1;
  }
  __syncthreads();
  if (tid < 2 * kCand) {
    const int b = tid / kCand, sl = tid % kCand;
    int page;
    if (sl < 16) {
      page = s.rslot[b][sl];
      if (page < 0) page = sl;                      // anchor page stands in (never legal)
    } else {
      page = s.aslot[b][sl - 16];
      if (page < 0) page = s.spare[b][sl - 16];     // spare unselected page (never legal)
    }
    if (page >= 0) s.slot[b][page] = (int8_t)sl;
    if (b < nrow) {
      int32_t* po = p.pool + ((long long)hs * p.T + t0 + b) * kPoolInts;
      po[sl] = page;
      if (sl < 16) {
        uint32_t bits = 0u;
        if (s.rslot[b][sl] >= 0) {
          const int part = sl >= 8;
          for (int j = part * 16; j < part * 16 + 16; ++j) bits |= (s.aslot[b][j] >= 0 ? 1u : 0u) << j;
        }
        po[kCand + sl] = (int32_t)bits;
      }
    }
  }

  // ---- probe operand, reader query u = Wq . probe (fp32)
  const int pi = lane & 31, hh = lane >> 5;
  const int blk = pi >> 4, m = pi & 15;
  const int tq = min(t0 + blk, p.T - 1);
  const long long row = p.gathered ? m : kProbeOffsets[m];
  const uint16_t* qbase = p.q + (long long)h * p.q_head + (long long)tq * p.q_block + row * p.q_row;
  u32x4 qop[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) qop[st] = ldg16(qbase + 64 * hh + 8 * st);
  {
    const int pr = tid >> 3, i = tid & 7;
    const int tb = min(t0 + (pr >> 4), p.T - 1);
    const long long rr = p.gathered ? (pr & 15) : kProbeOffsets[pr & 15];
    const uint16_t* qq = p.q + (long long)h * p.q_head + (long long)tb * p.q_block + rr * p.q_row;
    float acc = 0.f;
    for (int d = 0; d < 128; ++d) acc = fmaf(bf16_to_f32(qq[d]), p.wq[i * 128 + d], acc);
    s.u[pr][i] = acc;
  }

  const uint16_t* rkh = p.rk + (long long)h * p.HP * 4 * kHeadDim;
  const int ntiles = (P + 7) >> 3;
  const float inv_sqrt_d = 1.0f / sqrtf((float)kHeadDim);

  // ---- pass 1: LSE over all reps of each probe
  double mx = -INFINITY, sm = 0.0;
  for (int tile = wave; tile < ntiles; tile += 4) {
    f32x16 S;
    rep_tile(rkh, tile, P, lane, qop, S);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int page = tile * 8 + 2 * j + hh;
      if (page >= P) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const double z = (double)(S[4 * j + r] * inv_sqrt_d);
        if (z > mx) {
          sm = sm * exp(mx - z) + 1.0;
          mx = z;
        } else {
          sm += exp(z - mx);
        }
      }
    }
  }
  {
    const double om = __shfl_xor(mx, 32), os = __shfl_xor(sm, 32);
    const double mm = fmax(mx, om);
    const double tot = (mx == -INFINITY ? 0.0 : sm * exp(mx - mm)) + (om == -INFINITY ? 0.0 : os * exp(om - mm));
    if (hh == 0) {
      s.lse[wave][pi][0] = mm;
      s.lse[wave][pi][1] = tot;
    }
  }
  __syncthreads();
  double L;
  {
    double mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mm = fmax(mm, s.lse[w][pi][0]);
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      if (s.lse[w][pi][0] != -INFINITY) tot += s.lse[w][pi][1] * exp(s.lse[w][pi][0] - mm);
    L = mm + log(tot);
  }
  float u[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) u[i] = s.u[pi][i];

  // ---- pass 2: readout, summary approximation, mixtures, candidate endpoints
  double accH[16], accT[16], accB[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) accH[e] = accT[e] = accB[e] = 0.0;
  double sH = 0.0, sT = 0.0, sB = 0.0, lmax = -INFINITY;
  const long long row_id = ((long long)hs * p.T + tq) * 16 + m;
  for (int tile = wave; tile < ntiles; tile += 4) {
    f32x16 S;
    rep_tile(rkh, tile, P, lane, qop, S);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int page = tile * 8 + 2 * j + hh;
      if (page >= P) continue;
      float z[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = S[4 * j + r] * inv_sqrt_d;
      double w[4];
      const double lm = page_lse(z, w) - L;
      const double c0 = w[0] + w[1] - w[2] - w[3];
      const double c1 = w[0] - w[1] + w[2] - w[3];
      const double c2 = w[0] - w[1] - w[2] + w[3];
      // reader readout (fp32)
      const uint16_t* cf = p.coef + ((long long)h * p.EP + page) * kCoefStride;
      float co[88];
#pragma unroll
      for (int c = 0; c < 11; ++c) {
        const u32x4 v = ldg16(cf + 8 * c);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          co[8 * c + 2 * k] = bf16_lo(v[k]);
          co[8 * c + 2 * k + 1] = bf16_hi(v[k]);
        }
      }
      float A[32];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 v = ldg16(cf + kCoefA + 8 * c);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          A[8 * c + 2 * k] = bf16_lo(v[k]);
          A[8 * c + 2 * k + 1] = bf16_hi(v[k]);
        }
      }
      float F[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = fmaf(u[i], A[i * 4 + jj], acc);
        F[jj] = tanhf(acc);
      }
      float val[17];
#pragma unroll
      for (int k = 0; k < 17; ++k) {
        float acc = 0.f;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc = fmaf(F[jj], co[(jj + 1) * 17 + k], acc);
        val[k] = co[k] + acc;
      }
      const double beta = (double)val[16];
      const bool sel = s.sel[blk][page];
      const int sl = s.slot[blk][page];
      const double le = lm + beta;
      const double lg = sel ? le : lm;
      lmax = fmax(lmax, lg);
      const double ex = exp(lg), et = exp(le);
      sH += ex;
      sT += et;
      if (sl < 0) sB += ex;
      const double* mb = p.mean_b + ((long long)h * p.EP + page) * 16;
      const double* db = p.detail_b + ((long long)h * p.EP + page) * 48;
      double* cd = (sl >= 0 && blk < nrow) ? p.cand + (row_id * kCand + sl) * kCandVals : nullptr;
      if (cd) {
        cd[0] = lm;
        cd[1] = beta;
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const double ap = mb[e] + (c0 * db[e] + c1 * db[16 + e] + c2 * db[32 + e]);
        const double rp = (double)val[e];
        const double cur = sel ? ap + rp : ap;
        accH[e] += ex * cur;
        accT[e] += et * (ap + rp);
        if (sl < 0) accB[e] += ex * cur;
        if (cd) {
          cd[2 + e] = ap;
          cd[18 + e] = rp;
        }
      }
    }
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
  for (int i = tid; i < 32 * 16; i += 256) {
    const int pr = i >> 4, e = i & 15;
    const int b = pr >> 4;
    if (b >= nrow) continue;
    double aH = 0.0, aT = 0.0, aB = 0.0, zH = 0.0, zT = 0.0, zB = 0.0, lx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const double* pw = s.part[w][pr];
      aH += pw[e];
      aT += pw[16 + e];
      aB += pw[32 + e];
      zH += pw[48];
      zT += pw[49];
      zB += pw[50];
      lx = fmax(lx, pw[51]);
    }
    const double Hv = aH / zH;
    double* ro = p.rows + (((long long)hs * p.T + t0 + b) * 16 + (pr & 15)) * kRowVals;
    ro[e] = Hv;
    ro[16 + e] = aT / zT - Hv;
    ro[32 + e] = aB / zB;
    if (e == 0) {
      ro[48] = log(zB);
      ro[49] = lx;
      ro[50] = log(zH);
      ro[51] = 0.0;
    }
  }
}

// --------------------------------------------------------------- scores ----

struct ScoreSmem {
  double cand[kCand][kCandVals];
  double row[kRowVals];
  double rx[16], ro[16][16], ax[32], ao[32][16];
  float risk[kMaxPages];
  uint8_t sel[kMaxPages];
  int page[kCand];
  uint32_t legal[16];
  double best[4];
  int besti[4];
  int bad[4];
};

__device__ __forceinline__ double logaddexp(double a, double b) {
  if (a == -INFINITY) return b;
  if (b == -INFINITY) return a;
  const double mx = fmax(a, b);
  return mx + log1p(exp(-fabs(a - b)));
}

__global__ __launch_bounds__(256) void pset_scores_kernel(PsetParams p) {
  __shared__ ScoreSmem s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
  // pairs (i, j) = (tid / 32, tid % 32) and (8 + tid / 32, tid % 32)
  double acc[2] = {0.0, 0.0};
  for (int m = 0; m < 16; ++m) {
    __syncthreads();
    const double* cd = p.cand + (rowbase * 16 + m) * kCand * kCandVals;
    for (int i = tid; i < kCand * kCandVals; i += 256) (&s.cand[0][0])[i] = cd[i];
    if (tid < kRowVals) s.row[tid] = p.rows[(rowbase * 16 + m) * kRowVals + tid];
    __syncthreads();
    // leave-one-out groups (VR/scores.py:34-47): removes over er = lm + beta
    // with values c + rp, adds over la = lm with values c
    if (tid < kCand) {
      const bool rm = tid < 16;
      const int j = rm ? tid : tid - 16;
      const int k0 = rm ? 0 : 16, kn = rm ? 16 : 32;
      double mx = -INFINITY;
      for (int k = 0; k < kn; ++k) {
        if (k == j) continue;
        const double l = s.cand[k0 + k][0] + (rm ? s.cand[k0 + k][1] : 0.0);
        mx = fmax(mx, l);
      }
      double sum = 0.0, v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = 0.0;
      for (int k = 0; k < kn; ++k) {
        if (k == j) continue;
        const double l = s.cand[k0 + k][0] + (rm ? s.cand[k0 + k][1] : 0.0);
        const double w = exp(l - mx);
        sum += w;
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] += w * (s.cand[k0 + k][2 + e] + (rm ? s.cand[k0 + k][18 + e] : 0.0));
      }
      const double lse = mx + log(sum);
      if (rm) {
        s.rx[j] = lse;
#pragma unroll
        for (int e = 0; e < 16; ++e) s.ro[j][e] = v[e] / sum;
      } else {
        s.ax[j] = lse;
#pragma unroll
        for (int e = 0; e < 16; ++e) s.ao[j][e] = v[e] / sum;
      }
    }
    __syncthreads();
    const double lb = s.row[48], logmax = s.row[49];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = (tid >> 5) + 8 * q, j = tid & 31;
      const double* cr = s.cand[i];
      const double* ca = s.cand[16 + j];
      const double lr = cr[0], br = cr[1], er = lr + br;
      const double la = ca[0], ba = ca[1], ea = la + ba;
      double den = logaddexp(lb, s.rx[i]);
      den = logaddexp(den, s.ax[j]);
      den = logaddexp(den, lr);
      den = logaddexp(den, ea);
      // endpoint deltas; expm1 keeps beta near zero distinguishable
      const double xa = exp(ea - den), aa = exp(la - den);
      const double da = fabs(ba) < 0.5 ? aa * expm1(fmin(fmax(ba, -0.5), 0.5)) : xa - aa;
      const double xr = exp(er - den), ar = exp(lr - den);
      const double dr = fabs(br) < 0.5 ? ar * expm1(fmin(fmax(br, -0.5), 0.5)) : xr - ar;
      double delta[16];
      bool finite = true;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const double Hv = s.row[e];
        delta[e] = (da * (ca[2 + e] - Hv) + xa * ca[18 + e]) - (dr * (cr[2 + e] - Hv) + xr * cr[18 + e]);
        finite = finite && isfinite(delta[e]);
      }
      if (logmax - den > 80.0 || !finite) {
        const double wb = exp(lb - den), wrx = exp(s.rx[i] - den), wax = exp(s.ax[j] - den);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          double nw = wb * s.row[32 + e];
          nw += wrx * s.ro[i][e];
          nw += wax * s.ao[j][e];
          nw += ar * cr[2 + e];
          nw += xa * (ca[2 + e] + ca[18 + e]);
          delta[e] = nw - s.row[e];
        }
      }
      double ed = 0.0, dd = 0.0;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        ed += s.row[16 + e] * delta[e];
        dd += delta[e] * delta[e];
      }
      acc[q] += 2.0 * ed - dd;
    }
  }
  // legality, argmax (ties -> lowest pair index), finiteness
  double best = -INFINITY;
  int besti = 0x7fffffff;
  int bad = 0;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int i = (tid >> 5) + 8 * q, j = tid & 31;
    const int flat = i * 32 + j;
    double sc = acc[q] / 16.0;
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
    s.best[wave] = best;
    s.besti[wave] = besti;
    s.bad[wave] = bad;
  }
  __syncthreads();
  best = s.best[0];
  besti = s.besti[0];
  bad = s.bad[0];
  for (int w = 1; w < 4; ++w) {
    if (s.best[w] > best || (s.best[w] == best && s.besti[w] < besti)) {
      best = s.best[w];
      besti = s.besti[w];
    }
    bad += s.bad[w];
  }
  const bool exec = bad == 0 && best > 0.0;
  if (tid == 0) {
    p.gain[rowbase] = best;
    p.info[rowbase * 3 + 0] = exec ? 1 : 0;
    p.info[rowbase * 3 + 1] = besti;
    p.info[rowbase * 3 + 2] = bad;
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
  // LUT of the new selection: own first, then descending risk, ties -> lower page
  if (!p.ids) return;
  const int own = own_page(p, h, t);
  int32_t* ids = p.ids + ((long long)h * p.T + t) * p.C;
  if (tid == 0) ids[0] = own;
  for (int x = tid; x < P; x += 256) {
    if (!s.sel[x] || x == own) continue;
    const uint32_t kx = orderable(s.risk[x]);
    int rank = 0;
    for (int y = 0; y < P; ++y) {
      if (!s.sel[y] || y == own) continue;
      const uint32_t ky = orderable(s.risk[y]);
      rank += (ky > kx) || (ky == kx && y < x);
    }
    if (1 + rank < p.C) ids[1 + rank] = x;
  }
}

}  // namespace

extern "C" {

int ssa_encode(const void* keys, const void* mean, const void* detail, const void* stats, int head_pages,
               const void* basis, const float* w1t, const float* b1, const float* w2_reader, const float* b2_reader,
               const float* w2_phi, const float* b2_phi, const double* B, void* coef, double* mean_b,
               double* detail_b, int enc_pages, int heads, int first_page, int pages, int hidden,
               hipStream_t stream) {
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
  hipLaunchKernelGGL(encode_kernel, dim3((pages + kEncPages - 1) / kEncPages, heads), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

int ssa_pset(const void* q, long long q_head_stride, long long q_block_stride, long long q_row_stride,
             int gathered, const void* keys, int head_pages, const void* coef, const double* mean_b,
             const double* detail_b, int enc_pages, const float* wq, const float* risk, uint8_t* mask,
             int32_t* ids, const int32_t* own, const int32_t* heads, int n_heads, double* cand, double* rows,
             int32_t* pool, double* gain, int32_t* info, double* scores, int total_heads, int blocks, int pages,
             int count, hipStream_t stream) {
  if (n_heads <= 0 || n_heads > total_heads || blocks <= 0 || pages > kMaxPages || pages <= kAnchors + kCurrent ||
      head_pages < pages || enc_pages < pages || count < 1 || count > pages || pages - count < 64 ||
      heads == nullptr || cand == nullptr || rows == nullptr || pool == nullptr || gain == nullptr ||
      info == nullptr)
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
  p.H = total_heads;
  p.T = blocks;
  p.P = pages;
  p.C = count;
  const int np = (blocks + 1) / 2;
  hipLaunchKernelGGL(pset_rows_kernel, dim3(n_heads * np), dim3(256), 0, stream, p);
  hipLaunchKernelGGL(pset_scores_kernel, dim3(n_heads * blocks), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

}  // extern "C"
