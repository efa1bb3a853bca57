// Clean-commit token grouping for gfx950: the order in which a committed
// chunk's 4608 tokens fill its 72 pages (RV/runtime.py:57-68 GroupingOps.group).
//
//   features  f = (k - mean k).bank / sqrt(128) scaled to unit RMS, plus
//             0.1 tanh(gate) times the unit-RMS centred softmax response of
//             v.group_v                                  (LE/all_sparse_model.py:16-23)
//   balanced  7 levels of splits (3,3,2,2,2 over the chunk, then 2,2 inside
//             each page): each group is centred, a direction starts at the
//             one-hot of its highest-variance feature, takes 4 power steps,
//             and the group is stably sorted by its projection
//                                                        (LE/response_hard.py:20-31)
//   pages     a page permutation (Config.page_order, RV/ops.py:25-28)
//   chunk 0   a stable re-sort by frame, so the anchor frame fills pages
//             0..23                                      (VR/runtime.py:358-363)
//
// Everything after the bf16 inputs is fp64, so the order does not hinge on
// float32 rounding.  The batch is layers x heads independent rows b.
//   project_kernel   grid (72 token blocks, B): raw key and value projections
//   features_kernel  grid (B), 1024 threads: head-wide reductions, features
//   level_kernel     grid (B x groups): levels 0 and 1 (groups of 4608, 1536):
//                    stats, power steps, bitonic sort, rows through memory
//   fused_levels_kernel  grid (B x 9): levels 2..6 inside each 512-row group
//   frames_kernel    grid (B): the first chunk's stable partition by frame
#include "common.h"

using namespace ssa;

namespace {

constexpr int kTokens = 4608;      // 3 frames x 1536
constexpr int kFrame = 1536;
constexpr int kR = 32;             // feature width
constexpr int kPages = 72;
constexpr double kInvSqrtD = 11.313708498984761;   // sqrt(128), divided by as the reference does

struct GroupParams {
  const uint16_t* k;
  const uint16_t* v;
  long long layer_stride, tok_stride, head_stride;   // elements
  const float* bank;       // [B][32][128]
  const float* gv;         // [B][128][32]
  const float* gate;       // [B][32]
  const int32_t* page_dst; // [72] destination page of grouped page p, or null
  double* x[2];            // [B][4608][32] ping-pong
  int32_t* ids[2];         // [B][4608] ping-pong
  int32_t* order;          // [B][4608]
  int H, B;
};

__device__ __forceinline__ const uint16_t* row_ptr(const uint16_t* base, const GroupParams& p, int b, int t) {
  const int l = b / p.H, h = b % p.H;
  return base + (long long)l * p.layer_stride + (long long)t * p.tok_stride + (long long)h * p.head_stride;
}

// raw[b][t][r] = k_t . bank_r and vp[b][t][r] = v_t . gv[:, r] in fp64 (exact
// products of bf16 and fp32 values, summed in dimension order).  The 64
// tokens sit in LDS as bf16 rows (16-byte loads from memory), both weight
// matrices (gv transposed) as fp32 rows padded to 132 (16-byte reads,
// conflict-free across 16 consecutive rows): 68 KB, two workgroups per CU.
// Thread: tokens 4 tq .. 4 tq + 3 and features rp, rp + 16 of both
// projections, 16 fp64 accumulators.
constexpr int kRowPad = 132;
constexpr int kTokPad = 136;

__device__ __forceinline__ f32x4 bf16x4_to_f32(u32x2 w) {
  return f32x4{bf16_lo(w[0]), bf16_hi(w[0]), bf16_lo(w[1]), bf16_hi(w[1])};
}

__global__ __launch_bounds__(256, 2) void project_kernel(GroupParams p) {
  __shared__ alignas(16) uint16_t ks[64][kTokPad], vs[64][kTokPad];
  __shared__ alignas(16) float bk[kR][kRowPad], gvt[kR][kRowPad];
  const int blk = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  // 64 rows x 16 pieces of 16 bytes, for K and V
  for (int i = tid; i < 64 * 16; i += 256) {
    const int t = i >> 4, c = i & 15;
    *reinterpret_cast<u32x4*>(&ks[t][8 * c]) = ldg16(row_ptr(p.k, p, b, blk * 64 + t) + 8 * c);
    *reinterpret_cast<u32x4*>(&vs[t][8 * c]) = ldg16(row_ptr(p.v, p, b, blk * 64 + t) + 8 * c);
  }
  for (int i = tid; i < kR * kHeadDim / 4; i += 256) {
    const f32x4 w = reinterpret_cast<const f32x4*>(p.bank + (long long)b * kR * kHeadDim)[i];
    *reinterpret_cast<f32x4*>(&bk[(4 * i) / kHeadDim][(4 * i) % kHeadDim]) = w;
    const f32x4 g = reinterpret_cast<const f32x4*>(p.gv + (long long)b * kR * kHeadDim)[i];
    const int d = (4 * i) / kR, r = (4 * i) % kR;
#pragma unroll
    for (int c = 0; c < 4; ++c) gvt[r + c][d] = g[c];
  }
  __syncthreads();
  const int rp = tid & 15, tq = tid >> 4;
  double ak[4][2], av[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) ak[i][0] = ak[i][1] = av[i][0] = av[i][1] = 0.0;
  for (int d = 0; d < kHeadDim; d += 4) {
    f32x4 kk[4], vv[4], bb[2], gg[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kk[i] = bf16x4_to_f32(*reinterpret_cast<const u32x2*>(&ks[4 * tq + i][d]));
      vv[i] = bf16x4_to_f32(*reinterpret_cast<const u32x2*>(&vs[4 * tq + i][d]));
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bb[j] = *reinterpret_cast<const f32x4*>(&bk[rp + 16 * j][d]);
      gg[j] = *reinterpret_cast<const f32x4*>(&gvt[rp + 16 * j][d]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const double b0 = bb[0][c], b1 = bb[1][c], g0 = gg[0][c], g1 = gg[1][c];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const double kd = kk[i][c], vd = vv[i][c];
        ak[i][0] = fma(kd, b0, ak[i][0]);
        ak[i][1] = fma(kd, b1, ak[i][1]);
        av[i][0] = fma(vd, g0, av[i][0]);
        av[i][1] = fma(vd, g1, av[i][1]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const long long e = ((long long)b * kTokens + blk * 64 + 4 * tq + i) * kR + rp + 16 * j;
      p.x[0][e] = ak[i][j];
      p.x[1][e] = av[i][j];
    }
  }
}

// Sum of a per-thread value over the 32 threads sharing r (tid & 31) of a
// 1024-thread block; every thread gets the result.  red: 1024 doubles.
__device__ __forceinline__ double sum_over_tokens(double x, double* red, int tid) {
  red[tid] = x;
  __syncthreads();
  if (tid < 32) {
    double s = 0.0;
    for (int g = 0; g < 32; ++g) s += red[g * 32 + tid];
    red[1024 + tid] = s;
  }
  __syncthreads();
  const double s = red[1024 + (tid & 31)];
  __syncthreads();
  return s;
}

__device__ __forceinline__ double max_over_tokens(double x, double* red, int tid) {
  red[tid] = x;
  __syncthreads();
  if (tid < 32) {
    double s = -INFINITY;
    for (int g = 0; g < 32; ++g) s = fmax(s, red[g * 32 + tid]);
    red[1024 + tid] = s;
  }
  __syncthreads();
  const double s = red[1024 + (tid & 31)];
  __syncthreads();
  return s;
}

__device__ __forceinline__ double sum_all(double x, double* red, int tid) {
  const double s = sum_over_tokens(x, red, tid);   // per r
  red[tid] = s;
  __syncthreads();
  double t = 0.0;
  for (int r = 0; r < 32; ++r) t += red[r];
  __syncthreads();
  return t;
}

// Features of one row b (the head-wide reductions need the whole chunk):
// x[0] holds raw key projections on entry and the features on exit; x[1]
// the value projections; ids[0] = 0..4607.  Thread: r = tid & 31, tokens
// tid / 32 + 32 i.
__global__ __launch_bounds__(1024) void features_kernel(GroupParams p) {
  __shared__ double red[1024 + 32];
  const int b = blockIdx.x, tid = threadIdx.x, r = tid & 31, t0 = tid >> 5;
  double* raw = p.x[0] + (long long)b * kTokens * kR;
  const double* vp = p.x[1] + (long long)b * kTokens * kR;
  constexpr int kPer = kTokens / 32;
  double s = 0.0, mraw = -INFINITY;
  for (int i = 0; i < kPer; ++i) {
    const double x = raw[(t0 + 32 * i) * kR + r];
    s += x;
    mraw = fmax(mraw, x);
  }
  const double mean_raw = sum_over_tokens(s, red, tid) / kTokens;
  // score = centred key projection / sqrt(D).  Its max over t is the score
  // of the largest projection: (x - mean) / sqrt(D) rounds monotonically in
  // x, so this equals the max of the rounded scores bit for bit
  const double mx = (max_over_tokens(mraw, red, tid) - mean_raw) / kInvSqrtD;
  // one pass: the scores' RMS over (t, r), and the softmax over tokens
  // (denominator and sum of e * vp), each sum in token order
  double sq = 0.0, den = 0.0, num = 0.0;
  for (int i = 0; i < kPer; ++i) {
    const int e = (t0 + 32 * i) * kR + r;
    const double sc = (raw[e] - mean_raw) / kInvSqrtD;
    sq = fma(sc, sc, sq);
    const double ex = exp(sc - mx);
    den += ex;
    num = fma(ex, vp[e], num);
  }
  const double rms = fmax(sqrt(sum_all(sq, red, tid) / (kTokens * kR)), 1e-6);
  den = sum_over_tokens(den, red, tid);
  const double mean_a = sum_over_tokens(num, red, tid) / den;
  double sq2 = 0.0;
  for (int i = 0; i < kPer; ++i) {
    const int e = (t0 + 32 * i) * kR + r;
    const double a = exp((raw[e] - mean_raw) / kInvSqrtD - mx) / den;
    const double resp = a * kTokens * (vp[e] - mean_a);
    sq2 = fma(resp, resp, sq2);
  }
  const double rms2 = fmax(sqrt(sum_all(sq2, red, tid) / (kTokens * kR)), 1e-6);
  const double g = 0.1 * tanh((double)p.gate[b * kR + r]);
  for (int i = 0; i < kPer; ++i) {
    const int t = t0 + 32 * i, e = t * kR + r;
    const double sc = (raw[e] - mean_raw) / kInvSqrtD;
    const double a = exp(sc - mx) / den;
    const double resp = a * kTokens * (vp[e] - mean_a);
    raw[e] = sc / rms + g * (resp / rms2);
  }
  for (int t = tid; t < kTokens; t += 1024) p.ids[0][(long long)b * kTokens + t] = t;
}

// Ascending key of a double (-0.0 and +0.0 equal, as the sort compares them).
__device__ __forceinline__ unsigned long long order_key(double s) {
  if (s == 0.0) s = 0.0;
  const unsigned long long u = (unsigned long long)__double_as_longlong(s);
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

// Sum over the 8 lanes of a lane group (lanes 8q..8q+7).
__device__ __forceinline__ double sum8(double x) {
  x += xor_lane<1>(x);
  x += xor_lane<2>(x);
  x += xor_lane<4>(x);
  return x;
}

// One level of the balanced split: each workgroup takes one group of n rows
// of one b, in the current order (rows in[0..n) of the group), and writes
// them stably sorted by their projection on the power-iteration direction.
// Thread: features 4 q .. 4 q + 3 (q = tid & 7), rows tid / 8 + (THREADS / 8) i.
// The workgroup holds the group's sort keys in LDS and passes over its rows
// in memory seven times; THREADS / 64 waves keep that many row loads in
// flight.
template <int SORTN, int THREADS>
__global__ __launch_bounds__(THREADS) void level_kernel(GroupParams p, int n, int groups, int src) {
  constexpr int RS = THREADS / 8;   // row slots
  __shared__ unsigned long long key[SORTN];
  __shared__ unsigned short pos[SORTN];
  __shared__ double red[RS][kR + 1];
  __shared__ double vec[3][kR];   // mean, direction, scratch
  __shared__ int axis;
  const int tid = threadIdx.x, q = tid & 7, rs = tid >> 3;
  const int b = blockIdx.x / groups, gi = blockIdx.x % groups;
  const long long row0 = (long long)b * kTokens + (long long)gi * n;
  const double* x = p.x[src] + row0 * kR;
  const int32_t* ids = p.ids[src] + row0;
  auto reduce_rows = [&](const double (&a)[4], int slot) {
#pragma unroll
    for (int c = 0; c < 4; ++c) red[rs][4 * q + c] = a[c];
    __syncthreads();
    if (tid < kR) {
      double s = 0.0;
      for (int g = 0; g < RS; ++g) s += red[g][tid];
      vec[slot][tid] = s;
    }
    __syncthreads();
  };
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  for (int i = rs; i < n; i += RS) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] += x[(long long)i * kR + 4 * q + c];
  }
  reduce_rows(acc, 0);
  if (tid < kR) vec[0][tid] /= n;
  __syncthreads();
  double mean[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) mean[c] = vec[0][4 * q + c];
  // highest-variance feature (first of equals) -> one-hot start direction
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = 0.0;
  for (int i = rs; i < n; i += RS) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const double xc = x[(long long)i * kR + 4 * q + c] - mean[c];
      acc[c] = fma(xc, xc, acc[c]);
    }
  }
  reduce_rows(acc, 2);
  if (tid == 0) {
    int best = 0;
    double bv = vec[2][0] / n;
    for (int d = 1; d < kR; ++d) {
      const double vd = vec[2][d] / n;
      if (vd > bv) {
        bv = vd;
        best = d;
      }
    }
    axis = best;
  }
  __syncthreads();
  double dir[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) dir[c] = (4 * q + c == axis) ? 1.0 : 0.0;
  // 4 power steps: dir <- X_c^T (X_c dir), normalised (norm clamped at 1e-8)
  for (int it = 0; it < 4; ++it) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = 0.0;
    for (int i = rs; i < n; i += RS) {
      double xc[4], pr = 0.0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        xc[c] = x[(long long)i * kR + 4 * q + c] - mean[c];
        pr = fma(xc[c], dir[c], pr);
      }
      pr = sum8(pr);
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = fma(xc[c], pr, acc[c]);
    }
    reduce_rows(acc, 1);
    double nrm = 0.0;
    for (int d = 0; d < kR; ++d) nrm = fma(vec[1][d], vec[1][d], nrm);
    nrm = fmax(sqrt(nrm), 1e-8);
#pragma unroll
    for (int c = 0; c < 4; ++c) dir[c] = vec[1][4 * q + c] / nrm;
    __syncthreads();
  }
  // projections -> sort keys (ascending score, ties -> current position)
  for (int i = rs; i < SORTN; i += RS) {
    if (i < n) {
      double pr = 0.0;
#pragma unroll
      for (int c = 0; c < 4; ++c) pr = fma(x[(long long)i * kR + 4 * q + c] - mean[c], dir[c], pr);
      pr = sum8(pr);
      if (q == 0) {
        key[i] = order_key(pr);
        pos[i] = (unsigned short)i;
      }
    } else if (q == 0) {
      key[i] = ~0ull;
      pos[i] = 0xFFFF;
    }
  }
  __syncthreads();
  // A step of distance j <= 64 pairs elements within [2 e0, 2 e0 + 128) for
  // each aligned run e0 .. e0 + 63 of pairs, and wave w takes the same runs
  // (e0 = 64 w + THREADS m) in every step, so between two such steps it only
  // needs its own LDS writes before its reads; a workgroup barrier goes
  // before and after every step of a longer distance, and after the last.
  for (int kk = 2; kk <= SORTN; kk <<= 1) {
    for (int j = kk >> 1; j > 0; j >>= 1) {
      for (int e = tid; e < SORTN / 2; e += THREADS) {
        const int a = (e / j) * 2 * j + (e % j), c = a + j;
        const bool asc = (a & kk) == 0;
        const unsigned long long ka = key[a], kc = key[c];
        const unsigned short pa = pos[a], pc = pos[c];
        const bool greater = ka > kc || (ka == kc && pa > pc);
        if (greater == asc) {
          key[a] = kc;
          key[c] = ka;
          pos[a] = pc;
          pos[c] = pa;
        }
      }
      const int next = j > 1 ? j >> 1 : (2 * kk <= SORTN ? kk : 0);   // the next step's distance, 0: none
      if (j > 64 || next > 64 || next == 0) {
        __syncthreads();
      } else {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
  }
  double* xo = p.x[src ^ 1] + row0 * kR;
  int32_t* io = p.ids[src ^ 1] + row0;
  for (int j = rs; j < n; j += RS) {
    const int s = pos[j];
#pragma unroll
    for (int c = 0; c < 4; ++c) xo[(long long)j * kR + 4 * q + c] = x[(long long)s * kR + 4 * q + c];
    if (q == 0) io[j] = ids[s];
  }
}

// Levels 2..6 of the balanced split in one workgroup per 512-row group (a
// ninth of the chunk, as level 1 leaves it): the group's fp64 rows and token
// ids stay in LDS; level l sorts every aligned block of n = 512 >> (l - 2)
// rows by the block's own projection, all blocks at once, and a permutation
// of row slots carries the order from level to level.  Per block the steps
// and their arithmetic are level_kernel's.  Thread: features 4 q .. 4 q + 3
// (q = tid & 7), 8 rows of its block; the 512 / G threads of a block (G
// blocks) sum through LDS.  The last level writes the final order.
constexpr int kFuse = 512;
constexpr int kFuseLevels = 5;
constexpr int kFuseThreads = 512;
constexpr int kFuseGroups = kFuseThreads / 8;    // row groups of 8 threads
constexpr int kFuseRows = kFuse / kFuseGroups;   // rows per thread

__global__ __launch_bounds__(kFuseThreads, 1) void fused_levels_kernel(GroupParams p, int src, int32_t* last_out) {
  __shared__ alignas(16) double xs[kFuse][kR];   // 128 KB: rows in level 2's input order
  __shared__ unsigned short perm[2][kFuse];      // row slot at each position
  __shared__ int tok[kFuse];
  // the sums of the statistics and the sort keys are never live together
  __shared__ union {
    double red[kFuseGroups][kR + 1];
    struct {
      unsigned long long key[kFuse];
      unsigned short pos[kFuse];
    } s;
  } u;
  __shared__ double vec[2][kFuse / 32][kR];      // per block: mean | variance, then power-step sums
  __shared__ int axis[kFuse / 32];
  auto& red = u.red;
  auto& key = u.s.key;
  auto& pos = u.s.pos;
  const int tid = threadIdx.x, q = tid & 7, rg = tid >> 3;
  const int b = blockIdx.x / (kTokens / kFuse), gi = blockIdx.x % (kTokens / kFuse);
  const long long row0 = (long long)b * kTokens + (long long)gi * kFuse;
  {
    const f32x4* xsrc = reinterpret_cast<const f32x4*>(p.x[src] + row0 * kR);
    f32x4* xdst = reinterpret_cast<f32x4*>(&xs[0][0]);
    for (int e = tid; e < kFuse * kR / 2; e += kFuseThreads) xdst[e] = xsrc[e];
    for (int i = tid; i < kFuse; i += kFuseThreads) {
      tok[i] = p.ids[src][row0 + i];
      perm[0][i] = (unsigned short)i;
    }
  }
  __syncthreads();
  int cur = 0;
  for (int lv = 0; lv < kFuseLevels; ++lv) {
    const int n = kFuse >> lv, G = kFuse / n, T = kFuseThreads / G;   // block size, blocks, threads per block
    const int blk = tid / T, nrg = T >> 3, rgl = (tid % T) >> 3;
    const unsigned short* pm = perm[cur];
    // this thread's rows: positions blk * n + rgl + nrg * i, i < kFuseRows
    auto xrow = [&](int i) -> const double* { return xs[pm[blk * n + rgl + nrg * i]] + 4 * q; };
    // per-block sums of a per-thread partial over the block's row groups
    auto reduce_blocks = [&](const double (&a)[4], int slot) {
#pragma unroll
      for (int c = 0; c < 4; ++c) red[rg][4 * q + c] = a[c];
      __syncthreads();
      for (int e = tid; e < G * kR; e += kFuseThreads) {
        const int bb = e / kR, f = e % kR;
        double s = 0.0;
        for (int g = 0; g < nrg; ++g) s += red[bb * nrg + g][f];
        vec[slot][bb][f] = s;
      }
      __syncthreads();
    };
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int i = 0; i < kFuseRows; ++i) {
      const double* xr = xrow(i);
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] += xr[c];
    }
    reduce_blocks(acc, 0);
    double mean[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) mean[c] = vec[0][blk][4 * q + c] / n;
    // highest-variance feature (first of equals) -> one-hot start direction
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = 0.0;
    for (int i = 0; i < kFuseRows; ++i) {
      const double* xr = xrow(i);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const double xc = xr[c] - mean[c];
        acc[c] = fma(xc, xc, acc[c]);
      }
    }
    reduce_blocks(acc, 1);
    if (tid < G) {
      int best = 0;
      double bv = vec[1][tid][0] / n;
      for (int d = 1; d < kR; ++d) {
        const double vd = vec[1][tid][d] / n;
        if (vd > bv) {
          bv = vd;
          best = d;
        }
      }
      axis[tid] = best;
    }
    __syncthreads();
    double dir[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) dir[c] = (4 * q + c == axis[blk]) ? 1.0 : 0.0;
    for (int it = 0; it < 4; ++it) {
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = 0.0;
      for (int i = 0; i < kFuseRows; ++i) {
        const double* xr = xrow(i);
        double xc[4], pr = 0.0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          xc[c] = xr[c] - mean[c];
          pr = fma(xc[c], dir[c], pr);
        }
        pr = sum8(pr);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = fma(xc[c], pr, acc[c]);
      }
      reduce_blocks(acc, 1);
      double nrm = 0.0;
      for (int d = 0; d < kR; ++d) nrm = fma(vec[1][blk][d], vec[1][blk][d], nrm);
      nrm = fmax(sqrt(nrm), 1e-8);
#pragma unroll
      for (int c = 0; c < 4; ++c) dir[c] = vec[1][blk][4 * q + c] / nrm;
      __syncthreads();
    }
    // projections -> sort keys (ascending score, ties -> current position)
    for (int i = 0; i < kFuseRows; ++i) {
      const double* xr = xrow(i);
      double pr = 0.0;
#pragma unroll
      for (int c = 0; c < 4; ++c) pr = fma(xr[c] - mean[c], dir[c], pr);
      pr = sum8(pr);
      if (q == 0) {
        const int at = blk * n + rgl + nrg * i;
        key[at] = order_key(pr);
        pos[at] = (unsigned short)at;
      }
    }
    __syncthreads();
    // bitonic stages up to size n: every aligned block of n sorts on its own,
    // ascending (the direction bit of the last stage is masked to the block);
    // threads 0..255 each take one compare-exchange.  A step of distance
    // j <= 64 pairs elements within [128 w, 128 w + 128) for the pairs
    // e = 64 w .. 64 w + 63 of wave w, so between two such steps the wave only
    // needs its own LDS writes before its reads; a workgroup barrier goes
    // before and after every step of a longer distance, and after the last
    for (int kk = 2; kk <= n; kk <<= 1) {
      for (int j = kk >> 1; j > 0; j >>= 1) {
        const int e = tid & (kFuse / 2 - 1), a = (e / j) * 2 * j + (e % j), c = a + j;
        const bool asc = (a & kk & (n - 1)) == 0;
        const unsigned long long ka = key[a], kc = key[c];
        const unsigned short pa = pos[a], pc = pos[c];
        const bool greater = ka > kc || (ka == kc && pa > pc);
        if (tid < kFuse / 2 && greater == asc) {
          key[a] = kc;
          key[c] = ka;
          pos[a] = pc;
          pos[c] = pa;
        }
        const int next = j > 1 ? j >> 1 : (2 * kk <= n ? kk : 0);   // the next step's distance, 0: none
        if (j > 64 || next > 64 || next == 0) {
          __syncthreads();
        } else {
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
      }
    }
    for (int i = tid; i < kFuse; i += kFuseThreads) perm[cur ^ 1][i] = pm[pos[i]];
    cur ^= 1;
    __syncthreads();
  }
  // final order: position j is grouped page (gi * 512 + j) / 64, row j % 64
  for (int j = tid; j < kFuse; j += kFuseThreads) {
    const int in_head = gi * kFuse + j, page = in_head / 64;
    const int dpage = p.page_dst ? min(max(p.page_dst[page], 0), kPages - 1) : page;   // clamped: memory safety
    last_out[(long long)b * kTokens + dpage * 64 + in_head % 64] = tok[perm[cur][j]];
  }
}

// Stable partition of each row's order by frame (token / 1536): the first
// chunk's anchor frame fills pages 0..23 (VR/runtime.py:358-363).
__global__ __launch_bounds__(256) void frames_kernel(const int32_t* in, int32_t* out) {
  __shared__ int wsum[4];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int32_t* src = in + (long long)b * kTokens;
  int32_t* dst = out + (long long)b * kTokens;
  int cursor = 0;
  for (int f = 0; f < 3; ++f) {
    for (int c0 = 0; c0 < kTokens; c0 += 256) {
      const int val = src[c0 + tid];
      const bool on = val / kFrame == f;
      const unsigned long long bal = __ballot(on);
      if (lane == 0) wsum[w] = __popcll(bal);
      __syncthreads();
      int off = cursor;
      for (int u = 0; u < w; ++u) off += wsum[u];
      if (on) dst[off + __popcll(bal & ((1ull << lane) - 1ull))] = val;
      cursor += wsum[0] + wsum[1] + wsum[2] + wsum[3];
      __syncthreads();
    }
  }
}

}  // namespace

extern "C" {

int ssa_group_order(const void* k, const void* v, long long layer_stride, long long token_stride,
                    long long head_stride, const float* bank, const float* group_v, const float* gate,
                    const int32_t* page_dst, int first_chunk, int layers, int heads, double* scratch_x,
                    int32_t* scratch_ids, int32_t* order, hipStream_t stream) {
  if (layers <= 0 || heads <= 0 || !k || !v || !bank || !group_v || !gate || !scratch_x || !scratch_ids || !order ||
      layer_stride < 0 || token_stride < 0 || head_stride < 0)
    return (int)hipErrorInvalidValue;
  // rows are read 16 bytes at a time
  if ((((uintptr_t)k | (uintptr_t)v | (uintptr_t)bank | (uintptr_t)group_v) & 15) != 0 ||
      ((layer_stride | token_stride | head_stride) & 7) != 0)
    return (int)hipErrorInvalidValue;
  GroupParams p;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.layer_stride = layer_stride;
  p.tok_stride = token_stride;
  p.head_stride = head_stride;
  p.bank = bank;
  p.gv = group_v;
  p.gate = gate;
  p.page_dst = page_dst;
  p.H = heads;
  p.B = layers * heads;
  const long long rows = (long long)p.B * kTokens;
  p.x[0] = scratch_x;
  p.x[1] = scratch_x + rows * kR;
  p.ids[0] = scratch_ids;
  p.ids[1] = scratch_ids + rows;
  p.order = order;
  hipLaunchKernelGGL(project_kernel, dim3(kTokens / 64, p.B), dim3(256), 0, stream, p);
  hipLaunchKernelGGL(features_kernel, dim3(p.B), dim3(1024), 0, stream, p);
  // levels 0 and 1 (4608 -> 3 x 1536 -> 9 x 512) through global memory,
  // buffers 0 -> 1 -> 0; levels 2..6 inside each 512-row group, which
  // writes the order (or the frame partition's input)
  int32_t* last_out = first_chunk ? p.ids[1] : order;
  hipLaunchKernelGGL((level_kernel<8192, 1024>), dim3(p.B), dim3(1024), 0, stream, p, kTokens, 1, 0);
  hipLaunchKernelGGL((level_kernel<2048, 512>), dim3(p.B * 3), dim3(512), 0, stream, p, kTokens / 3, 3, 1);
  hipLaunchKernelGGL(fused_levels_kernel, dim3(p.B * (kTokens / kFuse)), dim3(kFuseThreads), 0, stream, p, 0,
                     last_out);
  if (first_chunk) hipLaunchKernelGGL(frames_kernel, dim3(p.B), dim3(256), 0, stream, p.ids[1], order);
  return (int)hipGetLastError();
}

}  // extern "C"
