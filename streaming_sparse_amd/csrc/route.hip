// Page router for gfx950: probe logits, row normaliser, risk and the page
// table, fused in one kernel per (head, pair of query blocks).
//
// Reference path (intersection tier, VB/graph.py:102-211):
//   z    = bf16(probe) . bf16(repK)^T * D^-1/2           (VR/tensor_bmm.py:56-66)
//   norm = max / sum exp over the P*4 reps of each probe  (VR/risk_online.py:88-113)
//   risk = mean over 16 probes of ((t0 x0 + t1 x1) + t2 x2) + t3 x3
//          (VR/runtime.py:27-40; kernels VR/risk_online.py:24-59,77-86),
//          here summed as (t0 x0 + t1 x1) + c sum_r prob_r W_r, the two
//          terms linear in the probabilities folded into one coefficient
//          per rep that a matrix product forms
//   mask = quota selection (VB/quota_mask.py:7-39) or the base LUT
//          (VR/runtime.py:279-288) or fixed top-k (VR/fixed_page_select.py:8-47)
//   ids  = own first, then descending risk                (VB/graph.py:210)
//
// Workgroup: 256 threads (4 waves) = 32 probes (2 query blocks) of one head.
// Each wave takes every 4th tile of 32 reps (8 pages).  S^T = R . Probe^T runs
// on v_mfma_f32_32x32x16_bf16, so a lane holds one probe and the 4 reps of
// each of its pages: the page's features are lane-local.  One pass over the
// reps: each lane keeps a running max and sum of exponentials of its probe,
// and since a page's features are linear in the probabilities of its reps,
// each page value is formed with 2^(z - running max) and rescaled once the
// probe's totals are known.  The rescaled values go through LDS to be summed
// over the 16 probes of a block; the risk rows then stay in LDS for the
// selection, a bitonic sort of 64-bit keys (group, orderable risk, ~page):
// ties -> lower page.  Workgroups appended to the grid write the call's rep
// value rows on the side.
#include "common.h"

using namespace ssa;

namespace {

constexpr int kThreads = 256;
constexpr int kMaxPages = 512;
constexpr int kAnchors = 24;
constexpr int kCurrent = 72;
constexpr int kTilesPerWave = kMaxPages / 32;   // tiles of 8 pages, every 4th to a wave

// Phase stamps of a measurement build (-DSSA_ROUTE_STAMPS, see
// streaming_sparse_amd/build.py): lane 0 of each wave of the first
// kStampBlocks workgroups records the shader clock (s_memtime, counted per
// XCD: only differences within one wave are meaningful) at the kernel's
// phase boundaries, read back by ssa_route_stamps.  The product library
// compiles the stamps out.
constexpr int kStampBlocks = 1024, kStampSlots = 16;
#ifdef SSA_ROUTE_STAMPS
__device__ unsigned long long route_stamps[kStampBlocks * 4 * kStampSlots];
#define ROUTE_STAMP(k)                                                                       \
  do {                                                                                       \
    if ((threadIdx.x & 63) == 0 && blockIdx.x < kStampBlocks)                                \
      route_stamps[(blockIdx.x * 4 + (threadIdx.x >> 6)) * kStampSlots + (k)] = __builtin_amdgcn_s_memtime(); \
  } while (0)
#else
#define ROUTE_STAMP(k) ((void)0)
#endif

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) const u32x2 lds_u32x2;
typedef __attribute__((address_space(3))) const uint16_t lds_u16;

struct RouteParams {
  const uint16_t* q;           // probe source
  long long q_head, q_block, q_row;   // element strides: head, query block, probe row
  int gathered;                // 1: q is [H,T,16,D] probes; 0: q is [1,N,H,D] queries
  const uint16_t* rk;          // rep keys [H, HP, 4, D]
  const uint16_t* stats;       // [H, HP, 4, 12]
  const float* theta;          // [H, 4]
  const int32_t* current;      // [H] current-page quota A (quota mode)
  const int32_t* own;          // [H, T] or null (own = P - T + t)
  float* risk;                 // [H, T, P]
  int32_t* ids;                // [H, T, C] or null
  uint8_t* mask;               // [H, T, P] or null
  float* lse;                  // [H, T, 16] LSE of each probe over all reps (natural log), or null
  int H, T, P, HP, C, mode, total;
  // detail operand tiles of the window, written on the side (rops null: not
  // asked for): detail [H,HP,3,8] bf16 -> rops [H,RT,kRepOpBytes/2] bf16
  const uint16_t* rdetail;
  uint16_t* rops;
  int RT;
  // near-tie report (tie_rows null: not asked for): rows h * T + t whose
  // selection boundary holds two risks within tie_eps relative, appended
  // to tie_rows through the counter *tie_count (zeroed by a launch before)
  float tie_eps;
  int32_t* tie_rows;
  int32_t* tie_count;
};

constexpr int kSlotBytes = 9 * 1024;   // a rep tile: 32 rows x 256 B (swizzled) + its pages' stats (768 B)

struct Sel {                   // selection state, aliasing the tile ring once the tiles are done
  unsigned long long key[2][kMaxPages];
  uint8_t sel[2][kMaxPages];
  int list[2][kMaxPages];
};

struct Smem {
  alignas(16) uint8_t ring[4][2][kSlotBytes];   // per-wave double buffer of rep tiles
  float part[4][32][2];        // per-wave (max, sum) of each probe
  float bmax[4];               // per-wave maximum of stats[p,1,11]
  float risk[2][kMaxPages];
};
static_assert(sizeof(Sel) <= sizeof(Smem::ring), "selection state must fit in the tile ring");

// Maxima as trees of v_max3 / v_max.  The sources build with NaN-free
// float semantics, so the compiler adds no quieting of matrix-pipe results
// (and keeps its own hazard waits before reading them).
__device__ __forceinline__ float max3f(float a, float b, float c) { return __builtin_fmaxf(__builtin_fmaxf(a, b), c); }
__device__ __forceinline__ float max2f(float a, float b) { return __builtin_fmaxf(a, b); }

// Rep tiles reach LDS by 16-byte global->LDS loads, 1 KB per wave
// instruction: load jj fills rows 4jj..4jj+3 of the tile, lane l the 16 bytes
// of row 4jj + l/16 at physical chunk l%16, which holds logical chunk
// (l%16) ^ (row & 15).  The MFMA operand reads (row lane%32, chunk 2st+hh)
// are then bank-conflict free.  Rows past the window re-read the last rep.
__device__ __forceinline__ uint32_t tile_row_off(int jj, int lane, int last_row) {
  const int row = 4 * jj + (lane >> 4);
  return (uint32_t)(min(row, last_row) * 256 + (((lane & 15) ^ (row & 15)) << 4));
}

// A operand of the tile in `slot`: rep row lane%32, dims 16*st + 8*hh + [0,8).
__device__ __forceinline__ void read_reps(const lds_u8* slot, int lane, u32x4 (&av)[8]) {
  const int r = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int st = 0; st < 8; ++st) av[st] = *(const lds_u32x4*)(slot + r * 256 + (((2 * st + hh) ^ (r & 15)) << 4));
}

__device__ __forceinline__ void rep_logits(const u32x4 (&av)[8], const u32x4 (&qop)[8], f32x16& S) {
  S = f32x16{};
#pragma unroll
  for (int st = 0; st < 8; ++st) S = mfma32(av[st], qop[st], S);
}

// Value of lane (lane ^ LX) for a 64-bit key: DPP quad permutes for 1 and 2,
// the DPP row rotate by 8 for 8, ds_swizzle bit-mask mode for 4 and 16, the
// 32-lane swap for 32.
template <int LX>
__device__ __forceinline__ uint32_t xlane32(uint32_t v, int lane) {
  if constexpr (LX == 1) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);   // [1,0,3,2]
  else if constexpr (LX == 2) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);   // [2,3,0,1]
  else if constexpr (LX == 8) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
  else if constexpr (LX == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return lane < 32 ? r[1] : r[0];
  } else {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (LX << 10) | 0x1F);
  }
}

template <int LX>
__device__ __forceinline__ unsigned long long xlane64(unsigned long long v, int lane) {
  const uint32_t lo = xlane32<LX>((uint32_t)v, lane), hi = xlane32<LX>((uint32_t)(v >> 32), lane);
  return ((unsigned long long)hi << 32) | lo;
}

// Descending bitonic sort of one row's 512 keys, held 4 per thread (element
// 4*bt + i in key[i]) by the row's 128 threads (two waves): partner distance
// 1 and 2 inside the thread, 4..128 by cross-lane shuffles inside the wave,
// 256 through LDS (`xchg`, the row's 512 slots) between the two waves.  Every
// thread of the workgroup calls it (both rows sort in lockstep; two barriers).
__device__ __forceinline__ void sort512_desc(unsigned long long (&key)[4], int bt, unsigned long long* xchg) {
#pragma unroll
  for (int k = 2; k <= kMaxPages; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j < 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (i & j) continue;
          const int e = 4 * bt + i;
          const bool desc = (e & k) == 0;
          const unsigned long long x = key[i], y = key[i | j];
          if ((x < y) == desc) {
            key[i] = y;
            key[i | j] = x;
          }
        }
      } else {
        unsigned long long other[4];
        if (j <= 128) {
          const int lane = bt & 63;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            switch (j) {
              case 4: other[i] = xlane64<1>(key[i], lane); break;
              case 8: other[i] = xlane64<2>(key[i], lane); break;
              case 16: other[i] = xlane64<4>(key[i], lane); break;
              case 32: other[i] = xlane64<8>(key[i], lane); break;
              case 64: other[i] = xlane64<16>(key[i], lane); break;
              default: other[i] = xlane64<32>(key[i], lane); break;
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) xchg[4 * bt + i] = key[i];
          __syncthreads();
#pragma unroll
          for (int i = 0; i < 4; ++i) other[i] = xchg[(4 * bt + i) ^ j];
          __syncthreads();
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 4 * bt + i;
          const bool desc = (e & k) == 0;
          const bool keep_max = ((e & j) == 0) == desc;
          const unsigned long long x = key[i], y = other[i];
          key[i] = (y > x) == keep_max ? y : x;
        }
      }
    }
  }
}

// Detail operand tiles written on the side by workgroups of their own,
// appended to the router's grid: they take the slots of the CUs that hold
// one router workgroup.  Thread c of block r writes chunk r * kThreads + c
// of the flat (head, tile, chunk) range.
__device__ void rep_operand_block(const RouteParams& p, int r) {
  const int tiles = (p.P + 15) >> 4;
  const int f = r * kThreads + threadIdx.x;
  if (f >= p.H * tiles * kRepOpChunks) return;
  const int c = f % kRepOpChunks, ht = f / kRepOpChunks, h = ht / tiles, rt = ht % tiles;
  const u32x4 w = rep_operand_chunk(p.rdetail + (long long)h * p.HP * 24, p.P, rt, c);
  *reinterpret_cast<u32x4*>(p.rops + ((long long)h * p.RT + rt) * (kRepOpBytes / 2) + 8 * c) = w;
}

__global__ __launch_bounds__(1) void zero_count_kernel(int32_t* count) { *count = 0; }

__global__ __launch_bounds__(kThreads, 2) void route_kernel(RouteParams p) {
  __shared__ Smem s;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int NP = (p.T + 1) >> 1;
  if ((int)blockIdx.x >= p.H * NP) {
    rep_operand_block(p, blockIdx.x - p.H * NP);
    return;
  }
  const int work = xcd_remap(blockIdx.x, p.H * NP);
  ROUTE_STAMP(0);
  const int h = work / NP, t0 = 2 * (work % NP);
  const int P = p.P;
  const int pi = lane & 31, hh = lane >> 5;
  const int blk = pi >> 4, m = pi & 15;

  const uint16_t* rkh = p.rk + (long long)h * p.HP * 4 * kHeadDim;
  const uint16_t* sth = p.stats + (long long)h * p.HP * 48;
  const int ntiles = (P + 7) >> 3;
  // logits in log2 units: z2 = q.k * log2(e) / sqrt(D); prob = 2^(z2 - max2) / den
  const float c2 = kLog2e / sqrtf((float)kHeadDim);
  // Each wave owns tiles wave + 4 j (j < nmine) and a double buffer of them
  // in LDS: no other wave reads its slots, so its own load counter orders
  // them.  A wave without tiles (P <= 24) re-reads the last tile and skips it.
  const int nmine = __builtin_amdgcn_readfirstlane(max((ntiles - wave + 3) >> 2, 0));
  auto mine = [&](int jj) { return min(wave + 4 * max(min(jj, nmine - 1), 0), ntiles - 1); };
  lds_u8* const ring = (lds_u8*)&s.ring[wave][0][0];
  const uint32_t ring_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)ring);
  // row offsets of a full tile in the instruction-offset form of dma_rows:
  // loads 0-3 and 4-7 each share one M0 value (rows >= 4 jj keep them >= 0)
  uint32_t koff[2][4];
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) koff[jj >> 2][jj & 3] = tile_row_off(jj, lane, 31) - 1024u * (jj & 3);
  // the stats of the tile's 8 pages: 768 contiguous bytes; lanes 48..63 land
  // past them in the slot's 1 KB stats region (a clamped re-read)
  auto issue_tile = [&](int tile_in, int slot, bool stats) {
    const int tile = __builtin_amdgcn_readfirstlane(tile_in);
    const uint32_t l = ring_addr + slot * kSlotBytes;
    const uint16_t* kb = rkh + (long long)tile * 32 * kHeadDim;
    const int last_row = P * 4 - 1 - tile * 32;
    if (last_row >= 31) {
      dma_rows<4>(kb, koff[0], l);
      dma_rows<4>(kb, koff[1], l + 4096);
    } else {
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) dma16(kb, tile_row_off(jj, lane, last_row), l + jj * 1024);
    }
    if (stats)
      dma16(sth + (long long)tile * 8 * 48, (uint32_t)min(16 * lane, (P - tile * 8) * 96 - 16), l + 8192);
  };
  // wait until at most n of this wave's global->LDS loads are outstanding
  auto wait_tile = [&](int n) {
    if (n == 8) __builtin_amdgcn_s_waitcnt(0x0F78);
    else __builtin_amdgcn_s_waitcnt(0x0F79);
  };
  auto wait_lds = [&]() { __builtin_amdgcn_s_waitcnt(0xC07F); };   // lgkmcnt(0)

  // Setup.  Every global read it needs is issued first and consumed before
  // the first rep tiles go out: the compiler's wait for one of these loads
  // would otherwise also wait for tile loads issued after it.
  //
  // probe rows: the workgroup's 32 probes (row r: block t0 + r / 16, probe
  // r % 16) go into this wave's ring slot 1 by 8 row-coalesced 1 KB loads,
  // 4 rows each with their chunks swizzled as a rep tile's (gathering each
  // lane's 16-byte operand pieces from global memory instead costs the
  // address unit one row per lane and load); slot 1 takes the wave's second
  // rep tile once the operand is read.
  {
    const uint16_t* qb = p.q + (long long)h * p.q_head + (long long)t0 * p.q_block;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int r = 4 * jj + (lane >> 4);
      const int dt = min(t0 + (r >> 4), p.T - 1) - t0;
      const long long prow = p.gathered ? (r & 15) : probe_row(r & 15);
      const int chunk = (lane & 15) ^ (r & 15);
      const uint32_t off = (uint32_t)(2 * (dt * p.q_block + prow * p.q_row + 8 * chunk));
      dma16(qb, off, ring_addr + kSlotBytes + jj * 1024);
    }
  }
  // max_p stats[p,1,11] over the head's pages: wave w reads pages
  // 128 w + lane and 128 w + 64 + lane (pages <= 512), the workgroup
  // combines the four partial maxima in LDS before the tiles (each page's
  // value is a lone 2-byte word, so a wave's loads cost the address unit one
  // cache line per lane: reading every page in every wave queued 8 such
  // loads per wave behind one another)
  uint32_t bw[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int pg = 128 * wave + 64 * i + lane;
    bw[i] = pg < P ? sth[(long long)pg * 48 + 23] : 0xff80u;
  }
  auto uniform = [](float v) { return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v))); };
  const float th0 = uniform(p.theta[h * 4 + 0]), th1 = uniform(p.theta[h * 4 + 1]);
  const float th2 = uniform(p.theta[h * 4 + 2]), th3 = uniform(p.theta[h * 4 + 3]);
  // the selection's inputs, requested here so that their latency overlaps
  // the setup's: the own page of the two blocks and the head's current quota
  int own_raw[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int tb = min(t0 + q, p.T - 1);
    own_raw[q] = __builtin_amdgcn_readfirstlane(p.own ? p.own[(long long)h * p.T + tb] : P - p.T + tb);
  }
  const int cur_raw = __builtin_amdgcn_readfirstlane(p.mode == 1 && P != kCurrent ? p.current[h] : p.total);
  asm volatile("" ::"s"(own_raw[0]), "s"(own_raw[1]), "s"(cur_raw));
  // the loads above are complete past this point
#pragma unroll
  for (int i = 0; i < 2; ++i) asm volatile("" ::"v"(bw[i]));
  wait_loads();
  ROUTE_STAMP(1);   // the setup's loads are in
  // probe operand (B): dims 16*st + 8*hh + [0,8) of probe pi, the k order of
  // read_reps
  u32x4 qop[8];
  read_reps(ring + kSlotBytes, lane, qop);
  wait_lds();
  // the first two rep tiles are in flight during the rest of the setup
  issue_tile(mine(0), 0, true);
  issue_tile(mine(1), 1, true);

  // q2[g] = sum of q^2 over dims 16g..16g+15 / D: this lane's 8 of them plus
  // the other lane half's
  float q2[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    float part = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float a = bf16_lo(qop[st][w]), b = bf16_hi(qop[st][w]);
      part += a * a + b * b;
    }
    const float other = xor_lane<32>(part);
    q2[st] = (part + other) / kHeadDim;
  }
  float qsum = 0.f;
#pragma unroll
  for (int g = 0; g < 8; ++g) qsum += q2[g];
  const float qn = sqrtf(qsum * kHeadDim) / sqrtf((float)kHeadDim);

  float bmax = wave_reduce(fmaxf(bf16_to_f32(bw[0]), bf16_to_f32(bw[1])), [](float a, float b) { return fmaxf(a, b); });
  if (lane == 0) s.bmax[wave] = bmax;
  __syncthreads();
  bmax = fmaxf(fmaxf(s.bmax[0], s.bmax[1]), fmaxf(s.bmax[2], s.bmax[3]));

  // One pass over the reps.  Each lane keeps a running max m and sum of
  // exponentials den of its probe over its reps; the features of a page are
  // linear in the probabilities of its reps, so each page value is formed
  // with 2^(z2 - m) and rescaled by 2^(m - MX) / DEN once the totals are
  // known.  Page values and the max they were formed with stay in registers.
  // B operands of the per-rep products, each value as two bf16 terms (the
  // hi parts in the lanes of k 0..7, the lo parts in those of k 8..15, or
  // hi | lo in one word):
  //   bq  = q2_g            against st[r, 0..7]        -> U = u_r
  //   bq3 = theta3 q2_g     against st[r, 0..7], and
  //   bwt = (theta2 qn, theta3 qn^2) against (st8, st8^2) -> W = theta2 beta + theta3 (u + beta^2)
  //   bone = 1              against st9 or st10         -> their broadcast
  u32x4 bq, bq3, bwt, bone;
  {
    auto rnd = [](float x) { return bf16_lo(pack_bf16(x, 0.f)); };
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float a = q2[2 * w], b = q2[2 * w + 1], a3 = th3 * a, b3 = th3 * b;
      bq[w] = hh == 0 ? pack_bf16(a, b) : pack_bf16(a - rnd(a), b - rnd(b));
      bq3[w] = hh == 0 ? pack_bf16(a3, b3) : pack_bf16(a3 - rnd(a3), b3 - rnd(b3));
    }
    const float w2 = th2 * qn, w3 = th3 * (qn * qn), w2h = rnd(w2), w3h = rnd(w3);
    bwt = hh == 0 ? u32x4{pack_bf16(w2h, w2 - w2h), pack_bf16(w3h, w3 - w3h), pack_bf16(w3h, 0.f), 0u} : u32x4{};
    bone = u32x4{hh == 0 ? 0x3F80u : 0u, 0u, 0u, 0u};
  }
  struct TileStats {
    u32x2 w01, w23, w45;
    float s011[4], s111[4];
  };
  auto read_stats = [&](int j, TileStats& ts) {
    const lds_u8* slot = ring + (j & 1) * kSlotBytes;
    const lds_u8* sr = slot + 8192 + pi * 24;
    ts.w01 = *(lds_u32x2*)sr;
    ts.w23 = *(lds_u32x2*)(sr + 8);
    ts.w45 = *(lds_u32x2*)(sr + 16);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const lds_u16* sp = (lds_u16*)(slot + 8192) + (2 * jj + hh) * 48;
      ts.s011[jj] = bf16_to_f32(sp[11]);
      ts.s111[jj] = bf16_to_f32(sp[23]);
    }
  };
  auto next_tile = [&](int j, f32x16& S, TileStats& ts) {
    wait_tile(9);
    u32x4 av[8];
    read_reps(ring + (j & 1) * kSlotBytes, lane, av);
    read_stats(j, ts);
    wait_lds();
    issue_tile(mine(j + 2), j & 1, true);
    rep_logits(av, qop, S);
  };
  const uint32_t lo_only = hh == 0 ? 0xffffffffu : 0u;
  float mx = -INFINITY, den = 0.f;
  float vals[kTilesPerWave][4], mj[kTilesPerWave];
  ROUTE_STAMP(2);   // probe norms, B operands, first tiles issued
  auto soft = [&](f32x16 S, const TileStats& ts, int tile, float (&v4)[4], float& mt) {
    const u32x4 ag = {ts.w01[0], ts.w01[1], ts.w23[0], ts.w23[1]};
    const uint32_t st8 = ts.w45[0] & 0xffffu, st9 = ts.w45[0] >> 16, st10 = ts.w45[1] & 0xffffu;
    // st8^2 is exact in fp32 (a bf16 has 8 significant bits) and splits
    // exactly into a bf16 hi part and a bf16 remainder
    const float s8 = bf16_to_f32(st8), sq = s8 * s8, sqh = bf16_lo(pack_bf16(sq, 0.f));
    const uint32_t sqw = pack_bf16(sqh, sqh);
    const u32x4 aw = {(st8 | (st8 << 16)) & lo_only, sqw & lo_only, pack_bf16(sq - sqh, 0.f) & lo_only, 0u};
    const f32x16 U = mfma32(ag, bq, f32x16{});
    const f32x16 W = mfma32(ag, bq3, mfma32(aw, bwt, f32x16{}));
    const f32x16 F9 = mfma32(u32x4{st9 & lo_only, 0u, 0u, 0u}, bone, f32x16{});
    const f32x16 F10 = mfma32(u32x4{st10 & lo_only, 0u, 0u, 0u}, bone, f32x16{});
    if (tile * 8 + 8 > P) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int page = tile * 8 + 2 * (i >> 2) + hh;
        if (page >= P) S[i] = -INFINITY;
      }
    }
    const float tmax = max2f(max3f(max3f(S[0], S[1], S[2]), max3f(S[3], S[4], S[5]), max3f(S[6], S[7], S[8])),
                             max3f(max3f(S[9], S[10], S[11]), max3f(S[12], S[13], S[14]), S[15]));
    const float mnew = fmaxf(mx, tmax * c2);
    float asum = 0.f;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      float prob[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) prob[i] = __builtin_amdgcn_exp2f(fmaf(S[4 * jj + i], c2, -mnew));
      const float alpha = ((prob[0] + prob[1]) + prob[2]) + prob[3];
      asum += alpha;
      const float c = ts.s111[jj] + bmax;
      // x0, x1 as the reference forms them; theta2 x2 + theta3 x3 =
      // c sum_r prob_r W_r.  u = sum_g q2_g st_g >= 0 (slots 0..7 hold mean
      // squares), so sqrt(|u|) is the reference's sqrt(max(u, 0)).
      float x0 = alpha * ts.s011[jj], x1 = 0.f, xw = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x0 += fabsf(prob[i] - alpha * 0.25f) * F9[4 * jj + i];
        x1 += prob[i] * __builtin_amdgcn_sqrtf(fabsf(U[4 * jj + i])) * F10[4 * jj + i];
        xw += prob[i] * W[4 * jj + i];
      }
      v4[jj] = fmaf(c, xw, fmaf(x1, th1, x0 * th0));
    }
    den = den * __builtin_amdgcn_exp2f(mx - mnew) + asum;
    mx = mnew;
    mt = mnew;
  };
#pragma unroll
  for (int j = 0; j < kTilesPerWave; ++j) {
    if (j < nmine) {
      f32x16 S;
      TileStats ts;
      next_tile(j, S, ts);
      soft(S, ts, mine(j), vals[j], mj[j]);
    }
  }
  wait_loads();                                      // the ring takes the probe sums, then the selection
  ROUTE_STAMP(3);   // tiles done
  {
    const float omx = xor_lane<32>(mx), oden = xor_lane<32>(den);
    const float mm = fmaxf(mx, omx);
    const float mu = mm == -INFINITY ? 0.f : mm;   // a wave without tiles (P <= 24) has none
    den = den * __builtin_amdgcn_exp2f(mx - mu) + oden * __builtin_amdgcn_exp2f(omx - mu);
    mx = mm;
    if (hh == 0) {
      s.part[wave][pi][0] = mx;
      s.part[wave][pi][1] = den;
    }
  }
  __syncthreads();
  float MX = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) MX = fmaxf(MX, s.part[w][pi][0]);
  float DEN = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) DEN += s.part[w][pi][1] * __builtin_amdgcn_exp2f(s.part[w][pi][0] - MX);
  const float nlse = -(MX + __log2f(DEN));
  ROUTE_STAMP(4);   // probe totals
  if (p.lse && wave == 0 && hh == 0 && t0 + blk < p.T)
    p.lse[((long long)h * p.T + t0 + blk) * 16 + m] = (MX + __log2f(DEN)) * 0.69314718055994531f;
  // page values: rescaled into LDS by probe ([block][page][probe], the tile
  // ring is free now), then summed over the block's 16 probes
  float* const tr = reinterpret_cast<float*>(&s.ring[0][0][0]);
  constexpr int kTrBlock = kMaxPages * 16 + 32;    // +32 floats: the two blocks use disjoint banks
#pragma unroll
  for (int j = 0; j < kTilesPerWave; ++j) {
    if (j < nmine) {
      const float f = __builtin_amdgcn_exp2f(mj[j] + nlse);
      const int tile = mine(j);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int page = tile * 8 + 2 * jj + hh;
        if (page < P) tr[blk * kTrBlock + page * 16 + m] = vals[j][jj] * f;
      }
    }
  }
  __syncthreads();
  const int nrow = min(2, p.T - t0);
  ROUTE_STAMP(5);   // page values in LDS
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    for (int pg = tid; pg < P; pg += kThreads) {
      const f32x4* src = reinterpret_cast<const f32x4*>(tr + b * kTrBlock + pg * 16);
      const f32x4 v0 = src[0], v1 = src[1], v2 = src[2], v3 = src[3];
      const float sum = (((v0[0] + v0[1]) + (v0[2] + v0[3])) + ((v1[0] + v1[1]) + (v1[2] + v1[3]))) +
                        (((v2[0] + v2[1]) + (v2[2] + v2[3])) + ((v3[0] + v3[1]) + (v3[2] + v3[3])));
      const float val = sum * 0.0625f;
      s.risk[b][pg] = val;
      if (b < nrow) p.risk[((long long)h * p.T + t0 + b) * P + pg] = val;
    }
  }
  __syncthreads();
  if (p.mode < 0) return;
  ROUTE_STAMP(6);   // probe sums, risk rows written

  // ---------------------------------------------------------------- select
  Sel& sl = *reinterpret_cast<Sel*>(&s.ring[0][0][0]);
  // Row b is sorted by its 128 threads (tid / 128 = b), 512 64-bit keys,
  // descending.  Key = (group << 62) | (orderable risk << 30) | (1023 - page):
  // risk descending, ties -> lower page, and the group field orders the
  // partitions (base / top-k: one group).
  const int b = tid >> 7, bt = tid & 127;
  int own[2];
  // own pages outside the window are clamped into it (memory safety of the
  // per-page state; a valid own is in [0, P))
#pragma unroll
  for (int q = 0; q < 2; ++q) own[q] = min(max(own_raw[q], 0), P - 1);
  // Quota partitions (VB/quota_mask.py:18-31): anchors [0,24), history
  // [24,cur_lo), current [cur_lo,P).  With P == 72 the anchor frame is the
  // chunk's first frame (VB/graph.py:143-148): current = [24,72), no history,
  // and the current quota is the whole total.  Each partition keeps its
  // quota clamped to [0, its size], as _keep does: current min(A, 72),
  // history total - A (with the unclamped A, as quota_mask passes it).  The
  // listed pages can then number more or fewer than the table holds.
  const int cur_lo = P == kCurrent ? kAnchors : P - kCurrent;
  const int ncur = P - cur_lo, nhist = cur_lo - kAnchors;
  int A = 0, nh = 0;
  if (p.mode == 1) {
    const int araw = cur_raw;
    A = min(max(araw, 0), ncur);
    nh = min(max(p.total - araw, 0), nhist);
  }
  unsigned long long keys[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int pg = 4 * bt + i;
    unsigned long long key = 0ull;
    if (pg < P) {
      const unsigned long long ord = (unsigned long long)orderable(s.risk[b][pg]) << 30;
      const unsigned long long low = (unsigned long long)(1023 - pg);
      if (p.mode == 0) {
        if (pg >= kAnchors && pg != own[b]) key = (1ull << 62) | ord | low;
      } else if (p.mode == 1) {
        if (pg >= cur_lo) key = pg == own[b] ? (3ull << 62) - 1ull - (unsigned long long)pg   // own first in current
                                             : (2ull << 62) | ord | low;
        else if (pg >= kAnchors) key = (1ull << 62) | ord | low;
      } else {
        key = pg == own[b] ? ~0ull - (unsigned long long)pg : ((1ull << 62) | ord | low);   // own first
      }
    }
    keys[i] = key;
  }
  ROUTE_STAMP(7);   // sort keys
  sort512_desc(keys, bt, sl.key[b]);
  ROUTE_STAMP(8);   // sorted
#pragma unroll
  for (int i = 0; i < 4; ++i) sl.key[b][4 * bt + i] = keys[i];
  __syncthreads();
  // sl.key[b] sorted descending; the page of entry i is 1023 - (key & 1023)
  auto page_at = [&](int i) -> int { return 1023 - (int)(sl.key[b][i] & 1023ull); };
  ROUTE_STAMP(9);   // sorted keys in LDS
  const bool row_ok = b < nrow;
  if (p.tie_rows && bt == 0 && row_ok) {
    // Near ties at the selection boundaries, in the sorted runs of the
    // partitions: the last kept entry of a run against the first dropped
    // one, when both are ranked by risk (not the forced own page); flagged
    // iff |a - c| <= eps max(|a|, |c|).  Base: the candidates (pages >= 24
    // other than own), C - 25 kept; quota: the current run (own first when
    // inside it), A kept, and the history run after it, nh kept; top-k: all
    // pages (own first), C kept.  The reference's recheck lists such rows
    // (VR/csrc/risk_close.cu:35-79, VR/risk_recheck.py:86-123).
    auto risk_at = [&](int i) { return s.risk[b][page_at(i)]; };
    auto near = [&](int base, int len, int kept, bool forced_first) {
      if (kept < 1 || kept >= len || (forced_first && kept == 1)) return false;
      const float a = risk_at(base + kept - 1), c = risk_at(base + kept);
      return fabsf(a - c) <= p.tie_eps * fmaxf(fabsf(a), fabsf(c));
    };
    bool tie;
    if (p.mode == 0) {
      tie = near(0, P - kAnchors - (own[b] >= kAnchors ? 1 : 0), p.C - 1 - kAnchors, false);
    } else if (p.mode == 1) {
      tie = near(0, ncur, A, own[b] >= cur_lo) || near(ncur, nhist, nh, false);
    } else {
      tie = near(0, P, p.C, true);
    }
    if (tie) p.tie_rows[atomicAdd(p.tie_count, 1)] = h * p.T + t0 + b;
  }
  int32_t* idsrow = p.ids ? p.ids + ((long long)h * p.T + t0 + b) * p.C : nullptr;
  for (int pg = bt; pg < P; pg += 128) sl.sel[b][pg] = 0;
  __syncthreads();
  if (p.mode == 0) {
    // LUT = [own, 0..23, top C-25 candidates], already in order
    for (int i = bt; i < p.C; i += 128) {
      const int pg = i == 0 ? own[b] : (i <= kAnchors ? i - 1 : page_at(i - 1 - kAnchors));
      sl.sel[b][pg] = 1;
      if (row_ok && idsrow) idsrow[i] = pg;
    }
  } else if (p.mode == 2) {
    for (int i = bt; i < p.C; i += 128) {
      const int pg = page_at(i);
      sl.sel[b][pg] = 1;
      if (row_ok && idsrow) idsrow[i] = pg;
    }
  } else {
    // quota: current top A at sorted [0, A) (own first), history top nh at
    // sorted [ncur, ncur + nh), anchors; list them, then order the LUT by risk
    const int nlist = kAnchors + A + nh;    // <= P
    for (int i = bt; i < nlist; i += 128) {
      const int pg = i < A ? page_at(i) : (i < A + nh ? page_at(ncur + i - A) : i - A - nh);
      sl.list[b][i] = pg;
      sl.sel[b][pg] = 1;
    }
    __syncthreads();
    if (idsrow) {
      // The LUT is topk(C) of the risk masked to the listed pages with own at
      // +inf (VB/graph.py:210): own first even when its quota left it out
      // (then it is an extra entry and the lowest listed page falls off),
      // then descending risk, ties -> lower page; slots past the entries
      // are padding -1.  LUT slot = number of entries with a larger key.
      // The sorted keys are no longer needed, so the entries' keys take
      // their place.
      const bool own_listed = sl.sel[b][own[b]] != 0;
      const int nent = nlist + (own_listed ? 0 : 1);   // <= P
      for (int i = bt; i < nent; i += 128) {
        const int pg = i < nlist ? sl.list[b][i] : own[b];
        if (i >= nlist) sl.list[b][i] = pg;
        sl.key[b][i] = pg == own[b] ? ~0ull
                                    : ((unsigned long long)orderable(s.risk[b][pg]) << 32) | (uint32_t)(1023 - pg);
      }
      __syncthreads();
      for (int i = bt; i < nent; i += 128) {
        const unsigned long long kx = sl.key[b][i];
        int rank = 0;
#pragma unroll 8
        for (int j = 0; j < nent; ++j) rank += sl.key[b][j] > kx;
        if (row_ok && rank < p.C) idsrow[rank] = sl.list[b][i];
      }
      for (int i = nent + bt; i < p.C; i += 128)
        if (row_ok) idsrow[i] = -1;
    }
  }
  __syncthreads();
  if (p.mask) {
    for (int pg = bt; pg < P; pg += 128)
      if (row_ok) p.mask[((long long)h * p.T + t0 + b) * P + pg] = sl.sel[b][pg];
  }
  ROUTE_STAMP(10);  // table, near-tie report and mask written
}


// RouteOps.select (RV/ops.py:113-138) on caller-given scores: one
// workgroup of 128 threads per (head, block) row, 4 pages per thread, and the
// router's descending sort of 512 64-bit keys: own first, then the valid
// pages by descending score (ties -> lower page), invalid and absent pages
// last.  count = clamp(#eligible, 1, cap) with overflow the excess over cap
// (threshold mode: eligible = valid and score > threshold, own forced), or
// min(fixed_count, #valid) without overflow; ids = the first count pages,
// then -1 up to id_capacity; residual = the sum of the scores of the valid
// unselected pages.
struct SelectParams {
  const float* scores;     // [rows, P]
  const int32_t* own;      // [rows]
  const uint8_t* valid;    // [rows, P] or null: every page valid
  int32_t* ids;            // [rows, id_capacity]
  int32_t* counts;         // [rows]
  uint8_t* mask;           // [rows, P]
  int32_t* overflow;       // [rows]
  float* residual;         // [rows]
  int P, id_capacity, cap, fixed_count, use_threshold;
  float threshold;
};

// Sum over the 128 threads of a workgroup (two waves); every thread gets it.
template <typename T>
__device__ __forceinline__ T sum128(T x, T* part, int bt) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  if ((bt & 63) == 0) part[bt >> 6] = x;
  __syncthreads();
  const T s = part[0] + part[1];
  __syncthreads();
  return s;
}

__global__ __launch_bounds__(128) void select_kernel(SelectParams p) {
  __shared__ unsigned long long xchg[kMaxPages];
  __shared__ uint8_t sel[kMaxPages];
  __shared__ int ipart[2];
  __shared__ float fpart[2];
  const int row = blockIdx.x, bt = threadIdx.x;
  const float* sc = p.scores + (long long)row * p.P;
  const uint8_t* vl = p.valid ? p.valid + (long long)row * p.P : nullptr;
  // an own page outside the window is clamped into it (memory safety of the
  // per-page state; a valid own is in [0, P))
  const int own = min(max(p.own[row], 0), p.P - 1);
  unsigned long long keys[4];
  float sv[4];
  bool vv[4];
  int elig = 0, nvalid = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int pg = 4 * bt + i;
    unsigned long long key = 0ull;
    sv[i] = 0.f;
    vv[i] = false;
    if (pg < p.P) {
      const bool v = vl ? vl[pg] != 0 : true;
      const float x = sc[pg];
      sv[i] = x;
      vv[i] = v;
      if (pg == own) key = ~0ull - (unsigned long long)pg;   // top, and decodes to pg
      else if (v) key = (1ull << 62) | ((unsigned long long)orderable(x) << 30) | (unsigned long long)(1023 - pg);
      elig += ((v && x > p.threshold) || pg == own) ? 1 : 0;
      nvalid += v ? 1 : 0;
    }
    keys[i] = key;
    sel[pg] = 0;
  }
  elig = sum128(elig, ipart, bt);
  nvalid = sum128(nvalid, ipart, bt);
  sort512_desc(keys, bt, xchg);
#pragma unroll
  for (int i = 0; i < 4; ++i) xchg[4 * bt + i] = keys[i];
  __syncthreads();
  int count, over = 0;
  if (p.use_threshold) {
    count = min(max(elig, 1), p.cap);
    over = max(elig - p.cap, 0);
  } else {
    count = min(p.fixed_count, nvalid);
  }
  int32_t* idrow = p.ids + (long long)row * p.id_capacity;
  for (int i = bt; i < p.id_capacity; i += 128) {
    const int pg = i < count ? 1023 - (int)(xchg[i] & 1023ull) : -1;
    idrow[i] = pg;
    if (pg >= 0) sel[pg] = 1;
  }
  __syncthreads();
  float res = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int pg = 4 * bt + i;
    if (pg < p.P) {
      p.mask[(long long)row * p.P + pg] = sel[pg];
      if (vv[i] && !sel[pg]) res += sv[i];
    }
  }
  res = sum128(res, fpart, bt);
  if (bt == 0) {
    p.counts[row] = count;
    p.overflow[row] = over;
    p.residual[row] = res;
  }
}

}  // namespace

extern "C" {

// Phase stamps of the last ssa_route launch in a measurement build: copies
// [kStampBlocks, 4 waves, 16] uint64 into `out` (host memory, `bytes` >= its
// size) and returns 0; hipErrorNotSupported in the product library.
int ssa_route_stamps(void* out, long long bytes) {
#ifdef SSA_ROUTE_STAMPS
  if (out == nullptr || bytes < (long long)sizeof(route_stamps)) return (int)hipErrorInvalidValue;
  return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(route_stamps), sizeof(route_stamps));
#else
  (void)out;
  (void)bytes;
  return (int)hipErrorNotSupported;
#endif
}

// mode: -1 risk only; 0 base (own + 24 anchors + top C-25); 1 anchor/current/
// history quota with `total` = A+B non-anchor pages and current[h] = A;
// 2 fixed top-C with own forced.
int ssa_route(const void* q, long long q_head_stride, long long q_block_stride, long long q_row_stride,
              int gathered, const void* keys, const void* stats, const float* theta, const int32_t* current,
              const int32_t* own, float* risk, int32_t* ids, uint8_t* mask, float* lse, int heads, int blocks,
              int pages, int head_pages, int count, int mode, int total, const void* detail, void* rep_ops,
              int rep_tiles, float tie_eps, int32_t* tie_rows, int32_t* tie_count, hipStream_t stream) {
  if (heads <= 0 || blocks <= 0 || pages <= 0 || pages > kMaxPages || head_pages < pages || mode < -1 ||
      mode > 2)
    return (int)hipErrorInvalidValue;
  // the near-tie report needs a selection, its counter and a non-negative epsilon
  if (tie_rows && (mode < 0 || !tie_count || !(tie_eps >= 0.0f))) return (int)hipErrorInvalidValue;
  // the operand tiles move in 16-byte stores
  if (rep_ops && (!detail || rep_tiles < (pages + 15) / 16 || ((uintptr_t)rep_ops & 15)))
    return (int)hipErrorInvalidValue;
  if (mode >= 0 && (count < 1 || count > pages)) return (int)hipErrorInvalidValue;
  if (mode == 0 && (count < 1 + kAnchors || pages < kAnchors + kCurrent)) return (int)hipErrorInvalidValue;
  // quota mode: windows of 72 pages (the anchor frame inside the chunk) or
  // at least anchors + current; total <= P - 24 non-anchor pages
  if (mode == 1 && (total < 0 || count != kAnchors + total || (pages != kCurrent && pages < kAnchors + kCurrent) ||
                    (pages != kCurrent && current == nullptr)))
    return (int)hipErrorInvalidValue;
  RouteParams p;
  p.q = (const uint16_t*)q;
  p.q_head = q_head_stride;
  p.q_block = q_block_stride;
  p.q_row = q_row_stride;
  p.gathered = gathered;
  p.rk = (const uint16_t*)keys;
  p.stats = (const uint16_t*)stats;
  p.theta = theta;
  p.current = current;
  p.own = own;
  p.risk = risk;
  p.ids = ids;
  p.mask = mask;
  p.lse = lse;
  p.H = heads;
  p.T = blocks;
  p.P = pages;
  p.HP = head_pages;
  p.C = count;
  p.mode = mode;
  p.total = total;
  p.rdetail = (const uint16_t*)detail;
  p.rops = (uint16_t*)rep_ops;
  p.RT = rep_tiles;
  p.tie_eps = tie_eps;
  p.tie_rows = tie_rows;
  p.tie_count = tie_count;
  // the counter starts at zero: a fill kernel rather than a memset node, so
  // that a captured graph replays it
  if (tie_rows) hipLaunchKernelGGL(zero_count_kernel, dim3(1), dim3(1), 0, stream, tie_count);
  const int np = (blocks + 1) / 2;
  const int nrv = rep_ops ? (heads * ((pages + 15) / 16) * kRepOpChunks + kThreads - 1) / kThreads : 0;
  hipLaunchKernelGGL(route_kernel, dim3(heads * np + nrv), dim3(kThreads), 0, stream, p);
  return (int)hipGetLastError();
}


// RouteOps.select on given scores; see select_kernel.  use_threshold = 0:
// count = min(fixed_count, #valid).
int ssa_select(const float* scores, const int32_t* own, const uint8_t* valid, int rows, int pages, float threshold,
               int use_threshold, int fixed_count, int cap, int id_capacity, int32_t* ids, int32_t* counts,
               uint8_t* mask, int32_t* overflow, float* residual, hipStream_t stream) {
  if (rows <= 0 || pages <= 0 || pages > kMaxPages || id_capacity < 1 || cap < 1 || cap > id_capacity ||
      cap > pages || (!use_threshold && (fixed_count < 1 || fixed_count > id_capacity)) || !scores || !own ||
      !ids || !counts || !mask || !overflow || !residual)
    return (int)hipErrorInvalidValue;
  SelectParams p;
  p.scores = scores;
  p.own = own;
  p.valid = valid;
  p.ids = ids;
  p.counts = counts;
  p.mask = mask;
  p.overflow = overflow;
  p.residual = residual;
  p.P = pages;
  p.id_capacity = id_capacity;
  p.cap = cap;
  p.fixed_count = fixed_count;
  p.use_threshold = use_threshold;
  p.threshold = threshold;
  hipLaunchKernelGGL(select_kernel, dim3(rows), dim3(128), 0, stream, p);
  return (int)hipGetLastError();
}

}  // extern "C"
