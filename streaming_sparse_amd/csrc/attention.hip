// Fused exact-page attention + summary compensation + softmax-mass merge for
// gfx950 (one kernel), plus the detail-operand prep it reads.
//
// The reference computes, per (query block t, head h) (RV/tuned_attention.py:
// 20-81 and RV/runtime.py:107-133):
//   exact: online softmax over the LUT pages' 64-token K/V       -> (O_e, le)
//   tail : softmax over the reps of the unselected pages, weight of rep r of
//          page p = 2^(q.r/sqrt(D)*log2e); value mean_p + (sum_a HAAR[a,r]
//          detail_pa) . basis^T; log-mass lt = mx + log2(den) + 4      -> (O_t, lt)
//   merge: rho = 1/(1+2^(le-lt)); out = (1-rho) O_e + rho O_t
// which equals ONE softmax over the union of the exact tokens (logit s,
// value v) and the unselected reps (logit z + 4 in log2 units, value
// mean_p + code_r . basis^T).  This kernel runs that union softmax: it walks
// "units" of 64 keys -- first the C exact pages (rows of the resident
// [L,H,D] cache), then the rep tiles of 16 pages x 4 reps whose pages are not
// all selected -- with one running max/sum per query.  A rep tile's values
// are never formed: with w_pr its rep weights, its share of the numerator is
//   sum_p a_p mean_p + (sum_{p,a} b_pa detail_pa) . basis^T,
// a_p = sum_r w_pr, b_pa = sum_r HAAR[a,r] w_pr, so the tile costs one
// 8-page product against the page means and two (one bf16 term per weight)
// or three (two terms) rank-8 products into a per-query code accumulator,
// which meets the basis once at the end.
//
// Workgroup: 4 waves, 64 queries of one head.  Wave w: pair w/2 takes keys
// 32*pair..32*pair+31 of every unit, queries 32*(w%2)..+31.  Per unit:
//   * K and V rows go straight from memory into a double-buffered LDS ring
//     (16-byte global->LDS loads, no register staging); the next unit's
//     loads are in flight while the current one computes;
//   * S^T = K . Q^T on v_mfma_f32_32x32x16_bf16: a lane holds one query, so
//     the softmax state is lane-local;
//   * O^T += V^T . P^T with V^T read by the LDS transpose read
//     (ds_read_b64_tr_b16) from row-major V;
//   * the O/l rescale runs only when some lane's running max grows.
// The two key halves are merged through LDS at the end.
#include "common.h"

#include <atomic>

#include <type_traits>

using namespace ssa;

namespace {

constexpr int kThreads = 256;
constexpr int kMaxCount = 512;
constexpr int kMaxRepTiles = 32;   // pages <= 512 -> ceil(P/16) <= 32
constexpr int kBuf = 64 * 256;     // one 64-row x 128-dim bf16 tile (K or V)

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;

struct AttnParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* rk;     // rep keys    [H, HP, 4, D]
  const uint16_t* mean;   // page means  [H, HP, D]
  const uint16_t* basis;  // [H, D, 8]
  const uint16_t* rops;   // detail operand tiles [H, RT, kRepOpBytes / 2]
  const int32_t* ids;     // [H, T, C]
  uint16_t* out;
  long long kv_tok, kv_head;   // element strides of a K/V token row and a head
  long long q_tok, q_head;     // element strides of q / out
  int H, T, P, HP, RT, C;
  float scale_log2;            // log2(e) / sqrt(D)
  // Workgroups >= split_from (grid order; a workgroup holds NB tiles) run
  // as split_k pieces of their unit list, one workgroup each; a piece leaves
  // the unnormalised state of its tile g in
  // part[((wg - split_from) * split_k + piece) * NB + g] for merge_kernel.
  // split_from = H * T / NB: no split.
  float* part;
  int split_from, split_k;
};

// Per piece of a split tile: O [qw][dt * 4 + j][64 lanes][4] fp32 (the
// epilogue's lane layout), then m [qw][32] and l [qw][32].
constexpr int kPieceFloats = 2 * 16 * 64 * 4 + 2 * 64;

// Step stamps of a measurement build (-DSSA_ATTN_STAMPS, see
// streaming_sparse_amd/build.py): in the one-block kernels, lane 0 of each
// wave of the first kAStampWGs workgroups records the shader clock
// (s_memtime, counted per XCD: only differences within one wave are
// meaningful) into LDS and copies the record out at the end, read back by
// ssa_attn_stamps.  Record of a wave (uint64): 0 start, 1 unit list built,
// 2 prologue done, 3 paired steps done, 4 last units done, 5 key halves
// exchanged, 6 npages | nunits << 16 | ibeg << 32 | (end of the paired
// steps) << 48, 7 HW_ID | XCC_ID << 32; then per paired step k (unit ibeg + k)
// three stamps: step start (after the previous barrier), body and max update
// done, loads waited for (before the barrier).  The product library compiles
// the stamps out.
constexpr int kAStampWGs = 1024, kAStampSteps = 96, kAStampRec = 8 + 3 * kAStampSteps;
#ifdef SSA_ATTN_STAMPS
__device__ unsigned long long attn_stamps[kAStampWGs * 4 * kAStampRec];
#define ATTN_TICK(k) tick(k)
#define ATTN_STAMP(k, v) stamp(k, v)
#else
#define ATTN_TICK(k) ((void)0)
#define ATTN_STAMP(k, v) ((void)0)
#endif

// K tile: 16-byte chunk c of row r at chunk c ^ (r & 15).
__device__ __forceinline__ int k_off(int row, int chunk) { return row * 256 + ((chunk ^ (row & 15)) << 4); }
// V tile: chunk c of row r at chunk c ^ vswz(r & 3); keeps the transpose reads
// of 4 rows x 16 or 32 dims on distinct banks.
__device__ __forceinline__ int vswz(int row) { return (0xEA40 >> (4 * (row & 3))) & 15; }   // 0, 4, 10, 14
__device__ __forceinline__ int v_off(int row, int chunk) { return row * 256 + ((chunk ^ vswz(row)) << 4); }

// A unit is a page p >= 0, or a rep tile rt (pages 16 rt .. 16 rt + 15) as
// 0x80000000 | drop << 8 | rt, bit b of the 16-bit `drop` set when page
// 16 rt + b is selected or beyond the window (its reps are masked out).
__device__ __forceinline__ int rep_unit(int rt, uint32_t drop) { return (int)(0x80000000u | (drop << 8) | (uint32_t)rt); }
__device__ __forceinline__ int rep_tile(int e) { return e & 0xff; }
__device__ __forceinline__ uint32_t rep_drop(int e) { return ((uint32_t)e >> 8) & 0xffffu; }

// Per-lane byte offsets of this wave's 4 K and 4 V rows of a unit (wave w
// loads rows 16w..16w+15, 1 KB per instruction) for a row stride `rs`
// (elements) and rows clamped to `last`.  With `inst` set, load jj's offset
// leaves out the jj * 1024 that its instruction offset adds (that offset
// moves the LDS destination by the same amount); rows >= 4 jj and rs >= 128
// keep these offsets non-negative.
struct UnitOffsets {
  uint32_t k[4], v[4];
};

__device__ __forceinline__ UnitOffsets unit_offsets(int wave, int lane, long long rs, int last, int nb, bool inst) {
  UnitOffsets o;
  const int pc = lane & 15, rows = 16 / nb;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int row = rows * wave + 4 * jj + (lane >> 4);
    const uint32_t r = (uint32_t)(min(row, last) * rs);
    const uint32_t sub = inst ? 1024u * jj : 0u;
    o.k[jj] = 2u * (r + 8u * (uint32_t)(pc ^ (row & 15))) - sub;
    o.v[jj] = 2u * (r + 8u * (uint32_t)(pc ^ vswz(row))) - sub;
  }
  return o;
}

// Per-lane byte offsets of a rep tile's loads: the K rows (instruction-
// offset form, as unit_offsets) and, for the general call's waves 0 and 2,
// the mean row of V-slot row rho = lane / 16 of the wave's first 1 KB within
// the tile's first page pair: pair-local page 2 (lane / 16), its 16-byte
// chunk lane % 16 swizzled by rho % 4 = lane / 16 (rows rho + 4 and rho + 8
// repeat it and add one page, 256 bytes).
struct RepOffsets {
  uint32_t k[4];
  uint32_t mean;
};

__device__ __forceinline__ RepOffsets rep_offsets(int wave, int lane, int nb) {
  RepOffsets o;
  const UnitOffsets u = unit_offsets(wave, lane, kHeadDim, 63, nb, true);
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) o.k[jj] = u.k[jj];
  const int g = lane >> 4;
  o.mean = (uint32_t)((8 * (wave >> 1) + 2 * g) * 256 + 16 * ((lane & 15) ^ vswz(g)));
  return o;
}

// Where a workgroup's units come from: head h's K, V, rep key and page mean
// rows and detail operand tiles as byte pointers, and the byte stride of a
// page.
struct UnitSources {
  const uint8_t *k, *v, *rk, *mean, *rops;
  uint32_t page_bytes;
};

__device__ __forceinline__ UnitSources unit_sources(const AttnParams& p, int h) {
  UnitSources u;
  u.k = (const uint8_t*)(p.k + (long long)h * p.kv_head);
  u.v = (const uint8_t*)(p.v + (long long)h * p.kv_head);
  u.rk = (const uint8_t*)(p.rk + (long long)h * p.HP * 4 * kHeadDim);
  u.mean = (const uint8_t*)(p.mean + (long long)h * p.HP * kHeadDim);
  u.rops = (const uint8_t*)(p.rops + (long long)h * p.RT * (kRepOpBytes / 2));
  u.page_bytes = (uint32_t)(128 * p.kv_tok);
  return u;
}

// Byte offset of a rep tile's detail operands in its V slot (rows 16..31,
// which the mean rows leave free).
constexpr int kDetailOff = 16 * 256;

// Enqueue the global->LDS loads of the K rows (kv = 0) or V rows (kv = 1)
// of unit e (a page, or a rep tile) into `buf`: wave w of the 4*NB waves
// loads rows (16/NB) w .. (16/NB) w + 16/NB - 1.  page_off / rep_off are the
// instruction-offset forms of unit_offsets.  The V slot of a rep tile
// (general call only) holds instead the page means of each key pair twice,
// row rho (0..15) of the pair's 32-row half = pair-local page 2 (rho % 4) +
// rho / 8 (waves 0 and 2), and the tile's detail operands at kDetailOff
// (wave 1).
template <int NB, int KIND = 2>
__device__ __forceinline__ void issue_rows(const AttnParams& p, const UnitSources& src, int e, int kv, int wave,
                                           int lane, const UnitOffsets& page_off, const RepOffsets& rep_off,
                                           lds_u8* buf) {
  constexpr int kLoads = 4 / NB;    // 1 KB loads per wave
  const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)buf + wave * 1024 * kLoads);
  if (KIND == 0 || (KIND == 2 && e >= 0)) {
    dma_rows<kLoads>((kv ? src.v : src.k) + (uint32_t)e * src.page_bytes, kv ? page_off.v : page_off.k, l);
  } else if (kv == 0) {
    const int rt = rep_tile(e);
    const uint8_t* base = src.rk + (uint32_t)rt * (64 * 256);
    // rows of pages >= P re-read the last valid rep (masked in compute)
    const int last = p.P * 4 - rt * 64 - 1;
    if (last >= 63) {
      dma_rows<kLoads>(base, rep_off.k, l);
    } else {
      const UnitOffsets o = unit_offsets(wave, lane, kHeadDim, last, NB, false);
#pragma unroll
      for (int jj = 0; jj < kLoads; ++jj) dma16(base, o.k[jj], l + jj * 1024);
    }
  } else if constexpr (NB == 1) {
    const int rt = rep_tile(e);
    const int w = __builtin_amdgcn_readfirstlane(wave);
    if (w == 1) {
      // 64 chunks of 16 bytes, one per lane
      dma16(src.rops + (uint32_t)rt * kRepOpBytes, 16u * (uint32_t)lane, l);
    } else if (w != 3) {
      // rows rho and rho + 4 hold page pg, rows rho + 8 and rho + 12 page
      // pg + 1; pages >= P re-read page P - 1 (their weights are zero)
      const uint8_t* base = src.mean + (uint32_t)rt * 4096u;
      if (16 * rt + 16 <= p.P) {
        dma16(base, rep_off.mean, l);
        dma16(base, rep_off.mean, l + 1024);
        dma16(base + 256, rep_off.mean, l + 2048);
        dma16(base + 256, rep_off.mean, l + 3072);
      } else {
        const int pg = 16 * rt + 8 * (w >> 1) + 2 * (lane >> 4);
        const uint32_t cpart = rep_off.mean & 255u;
        const uint32_t o0 = (uint32_t)(min(pg, p.P - 1) - 16 * rt) * 256u + cpart;
        const uint32_t o1 = (uint32_t)(min(pg + 1, p.P - 1) - 16 * rt) * 256u + cpart;
        dma16(base, o0, l);
        dma16(base, o0, l + 1024);
        dma16(base, o1, l + 2048);
        dma16(base, o1, l + 3072);
      }
    }
  }
}

// V^T operand for O^T += V^T P^T: dims 32*dt + lane%32, keys (MFMA k order)
// 16*ks + 8*(e/4) + 4*hh + e%4 of this pair's half, from two transpose reads.
__device__ __forceinline__ u32x4 v_operand(const lds_u8* vbuf, int pair, int ks, int dt, int lane) {
  const int g = lane >> 4, i = lane & 15, hh = g >> 1;
  const int chunk = 4 * dt + 2 * (g & 1) + ((i & 3) >> 1);
  const int half = (i & 1) * 8;
  const int row0 = 32 * pair + 16 * ks + 4 * hh + (i >> 2);
  const bf16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(vbuf + v_off(row0, chunk) + half));
  const bf16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(vbuf + v_off(row0 + 8, chunk) + half));
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return u32x4{ua[0], ua[1], ub[0], ub[1]};
}

// Lane parts of the K and V operand read addresses within a slot.  K: the
// chunk 2 x + hh of row 32 pair + lane % 32 sits at k_base ^ (x << 5) (the
// swizzle XOR touches address bits 4..7 only).  V: the first transpose read
// of k step ks, dim tile dt sits at 4096 ks + (v_base ^ (dt << 6)), the
// second 8 rows (2048 bytes) further.  The loop bodies form the addresses
// from these two values, so that only they stay live across units.
__device__ __forceinline__ uint32_t k_base(int pair, int lane) {
  const int row = 32 * pair + (lane & 31);
  return (uint32_t)(row * 256 + (((lane >> 5) ^ (row & 15)) << 4));
}
__device__ __forceinline__ uint32_t v_base(int pair, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int row0 = 32 * pair + 4 * (g >> 1) + (i >> 2);
  const int c0 = 2 * (g & 1) + ((i & 3) >> 1);
  return (uint32_t)(row0 * 256 + ((c0 ^ vswz(row0)) << 4) + (i & 1) * 8);
}
__device__ __forceinline__ u32x4 k_read(const lds_u8* kb, uint32_t kl, int x) {
  return *(lds_u32x4*)(kb + (kl ^ (uint32_t)(x << 5)));
}
// the V^T operand of v_operand from the address base
__device__ __forceinline__ u32x4 v_read(const lds_u8* vb, uint32_t vl, int ks, int dt) {
  const lds_u8* a = vb + 4096 * ks + (vl ^ (uint32_t)(dt << 6));
  const bf16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)a);
  const bf16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(a + 2048));
  const u32x2 ux = __builtin_bit_cast(u32x2, x), uy = __builtin_bit_cast(u32x2, y);
  return u32x4{ux[0], ux[1], uy[0], uy[1]};
}

// S^T = K . Q^T for this pair's 32 keys of the unit in `kbuf`; S[i] is key
// 32*pair + 8*(i/4) + 4*hh + i%4, query lane%32.  All 8 K operands are read
// before the first MFMA.
__device__ __forceinline__ f32x16 s_tile(const lds_u8* kbuf, int pair, int lane, const u32x4 (&qop)[8]) {
  const int r = lane & 31, hh = lane >> 5;
  u32x4 a[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) a[st] = *(lds_u32x4*)(kbuf + k_off(32 * pair + r, 2 * st + hh));
  f32x16 S = {};
#pragma unroll
  for (int st = 0; st < 8; ++st) S = mfma32(a[st], qop[st], S);
  return S;
}

// Maxima as trees of v_max3 / v_max.  The sources build with NaN-free
// float semantics, so the compiler adds no quieting of matrix-pipe results
// (and keeps its own hazard waits before reading them).
__device__ __forceinline__ float max3f(float a, float b, float c) { return __builtin_fmaxf(__builtin_fmaxf(a, b), c); }
__device__ __forceinline__ float max2f(float a, float b) { return __builtin_fmaxf(a, b); }

// Row max of S in log2 units (+ bias); rep tiles first drop the reps of
// selected pages and of pages >= P.  Returns the bias of the unit.
template <int KIND = 2>
__device__ __forceinline__ float unit_max(f32x16& S, int e, int pair, int lane, float scale_log2, float& mloc) {
  float bias = 0.0f;
  if (KIND == 1 || (KIND == 2 && e < 0)) {
    bias = 4.0f;
    const uint32_t drop = rep_drop(e) >> (8 * pair + (lane >> 5));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool d = (drop >> (2 * j)) & 1u;
#pragma unroll
      for (int i = 0; i < 4; ++i) S[4 * j + i] = d ? -INFINITY : S[4 * j + i];
    }
  }
  // a depth-3 tree of v_max3 (S holds no NaN, so no operand quieting)
  const float a = max3f(S[0], S[1], S[2]), b = max3f(S[3], S[4], S[5]), c = max3f(S[6], S[7], S[8]);
  const float d = max3f(S[9], S[10], S[11]), e2 = max3f(S[12], S[13], S[14]);
  float mx = max2f(max3f(a, b, c), max3f(d, e2, S[15]));
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
  mx = max2f(__uint_as_float(sw[0]), __uint_as_float(sw[1]));   // max over lanes l and l ^ 32
  mloc = mx * scale_log2 + bias;     // -inf stays -inf
  return bias;
}

// Running-max update with a lazy threshold: the accumulator is rescaled only
// when some lane's unit max exceeds its running max by more than kSlack
// (log2 units), so probabilities stay below 2^kSlack and the rescale is rare.
constexpr float kSlack = 8.0f;

// The running max m of a lane.  With KEEP, two values are kept beside it,
// so that a step reads them instead of re-forming them: neg = -m (0 while
// m = -inf), the exponent offset of the probabilities, and thr = m +
// kSlack (2 VGPRs that the two-term general call has no room for; it
// re-forms them, with the same results).
template <bool KEEP>
struct RunMax {
  float m = -INFINITY, neg_ = 0.0f, thr_ = -INFINITY;
  __device__ __forceinline__ float neg() const { return KEEP ? neg_ : -(m == -INFINITY ? 0.0f : m); }
  __device__ __forceinline__ float thr() const { return KEEP ? thr_ : m + kSlack; }
};

// `ls` is a lane's fp32 partial denominator (the sum of the fp32
// probabilities of its keys, in either arithmetic, as the reference's l).
// C holds the code accumulator in items 0..3 (ranks 4 hh + i).
template <bool KEEP>
__device__ __forceinline__ void update_max(float mloc, RunMax<KEEP>& r, float& ls, f32x16 (&O)[4], f32x16& C) {
  if (__any(mloc > r.thr())) {
    const float mnew = fmaxf(r.m, mloc);
    const float mu = mnew == -INFINITY ? 0.0f : mnew;
    const float alpha = __builtin_amdgcn_exp2f(r.m - mu);
    ls *= alpha;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) O[dt] *= alpha;
#pragma unroll
    for (int i = 0; i < 4; ++i) C[i] *= alpha;
    r.m = mnew;
    if (KEEP) {
      r.neg_ = -mu;
      r.thr_ = mnew + kSlack;
    }
  }
}

// Word w of the two-term operands from two fp32 probabilities: hi = bf16(P)
// pairs, lo = bf16(P - bf16(P)) pairs (LE/gap_exact_round_kernel.py:110-125).
// The empty asm hands the packed word on opaquely: otherwise the compiler
// rebuilds bf16(p0) for the low half with a second conversion.
__device__ __forceinline__ u32x2 split_pair(float p0, float p1) {
  uint32_t hi = pack_bf16(p0, p1);
  asm volatile("" : "+v"(hi));
  return u32x2{hi, pack_bf16(p0 - bf16_lo(hi), p1 - bf16_hi(hi))};
}

// P = 2^(S*scale + nb) as the bf16 B operands of the two k steps (pb; pl =
// the low parts bf16(P - bf16(P)) for the two-term product); the
// denominator `ls` gathers the fp32 P of the lane in either arithmetic.
template <bool PRECISE>
__device__ __forceinline__ void probabilities(const f32x16& S, float nb, float scale_log2, u32x4 (&pb)[2],
                                              u32x4 (&pl)[2], float& ls) {
  float P[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) P[i] = __builtin_amdgcn_exp2f(fmaf(S[i], scale_log2, nb));
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int o = 8 * ks;
    pl[ks] = u32x4{};
    if (PRECISE) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const u32x2 hl = split_pair(P[o + 2 * w], P[o + 2 * w + 1]);
        pb[ks][w] = hl[0];
        pl[ks][w] = hl[1];
      }
    } else {
      pb[ks] = u32x4{pack_bf16(P[o + 0], P[o + 1]), pack_bf16(P[o + 2], P[o + 3]),
                     pack_bf16(P[o + 4], P[o + 5]), pack_bf16(P[o + 6], P[o + 7])};
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += P[i];
  ls += s;
}

// Haar view of one page's 4 rep probabilities w: hw = {a, b0, b1, b2}, the
// mean weight a = sum_r w_r and the contrast weights b_a = sum_r HAAR[a,r] w_r
// (HAAR rows (1,1,-1,-1), (1,-1,1,-1), (1,-1,-1,1); RV/ops.py:10).
__device__ __forceinline__ void haar4(const float* w, float* hw) {
  const float s01 = w[0] + w[1], s23 = w[2] + w[3], d01 = w[0] - w[1], d23 = w[2] - w[3];
  hw[0] = s01 + s23;
  hw[1] = s01 - s23;
  hw[2] = d01 + d23;
  hw[3] = d01 - d23;
}

// Exchange of lane halves (v_permlane32_swap): lanes l < 32 get {lo of lane
// l, lo of lane l + 32}, lanes l >= 32 get {hi of lane l - 32, hi of lane l}.
// A word of hi parts and one of lo parts, spread over the two halves of a
// query's lanes, so become the k = 8 hh .. 8 hh + 7 operand items of the
// half that holds that part for all of them.
__device__ __forceinline__ u32x2 halves(uint32_t lo, uint32_t hi) {
  const auto s = __builtin_amdgcn_permlane32_swap(lo, hi, false, false);
  return u32x2{s[0], s[1]};
}

// O^T += V^T P^T (two-term: hi and lo parts of P).
template <bool PRECISE>
__device__ __forceinline__ void pv(const u32x4 (&pb)[2], const u32x4 (&pl)[2], const lds_u8* vbuf, int pair,
                                   int lane, f32x16 (&O)[4]) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const u32x4 va = v_operand(vbuf, pair, ks, dt, lane);
      O[dt] = mfma32(va, pb[ks], O[dt]);
      if (PRECISE) O[dt] = mfma32(va, pl[ks], O[dt]);
    }
  }
}

// Unit list of tile (t, h): its exact pages in LUT order, then the rep tiles
// holding at least one page the table does not select (each carrying its
// drop mask); maskw gets the 512-bit page mask.  LUT entries outside [0, P)
// (the -1 padding of a shorter table) are not read: they add no exact unit
// and select nothing.  A page listed twice is attended twice, as a LUT walk
// does.  Called by every 4-wave workgroup's threads; wcount is 4 ints of LDS.
// first: this thread's entry of the table's first kThreads entries, read by
// the caller (lut_entry) before its other loads.
__device__ __forceinline__ int lut_entry(const AttnParams& p, int h, int t, int i) {
  return i < p.C ? p.ids[((long long)h * p.T + t) * p.C + i] : -1;
}

// STAGE 1 lists the exact pages only, STAGE 2 the rep tiles only (the two
// launches of a staged call); STAGE 0 both.
template <int STAGE>
__device__ void own_units(const AttnParams& p, int h, int t, int tid, int first, int* units, uint32_t* maskw,
                          int* wcount, int* nunits, int* nexact) {
  const int lane = tid & 63, wave = tid >> 6;
  if (tid < 16) maskw[tid] = 0u;
  __syncthreads();
  int base = 0;
  for (int i0 = 0; i0 < p.C; i0 += kThreads) {
    const int pg = i0 == 0 ? first : lut_entry(p, h, t, i0 + tid);
    const bool ok = pg >= 0 && pg < p.P;
    const unsigned long long bal = __ballot(ok);
    if (lane == 0) wcount[wave] = __popcll(bal);
    __syncthreads();
    int off = base;
    for (int w = 0; w < wave; ++w) off += wcount[w];
    if (ok) {
      if (STAGE != 2) units[off + __popcll(bal & ((1ull << lane) - 1ull))] = pg;
      atomicOr(&maskw[pg >> 5], 1u << (pg & 31));
    }
    base += wcount[0] + wcount[1] + wcount[2] + wcount[3];
    __syncthreads();
  }
  if (tid < 64) {
    const int R = (p.P + 15) >> 4;
    bool live = false;
    uint32_t drop = 0xffffu;
    if (lane < R) {
      const int p0 = lane * 16;
      const uint32_t word = (maskw[p0 >> 5] >> (p0 & 31)) & 0xffffu;
      const int valid = min(16, p.P - p0);
      const uint32_t vmask = valid >= 16 ? 0xffffu : ((1u << valid) - 1u);
      drop = (word | ~vmask) & 0xffffu;
      live = drop != 0xffffu;
    }
    const unsigned long long bal = __ballot(live);
    const int rbase = STAGE == 2 ? 0 : base;
    if (STAGE != 1 && live) units[rbase + __popcll(bal & ((1ull << lane) - 1ull))] = rep_unit(lane, drop);
    if (lane == 0) {
      *nunits = STAGE == 1 ? base : rbase + __popcll(bal);
      *nexact = STAGE == 2 ? 0 : base;
    }
  }
}

// NB query blocks per workgroup (4 waves each).  NB = 1: the general call
// (own page table, rep tiles).  NB = 2: a call that selects every page, so
// both blocks walk the same units (pages 0..P-1) and share each K/V load.
// STAGE (general call only): 0 walks every unit of a tile and writes out (or
// a piece's state); 1 and 2 are the two launches of a staged call -- the
// exact pages, then the compensation's rep tiles -- each leaving its state
// in part[2 tile + STAGE - 1] for merge_kernel, the reference's split into
// an exact kernel, a tail and a merge (RV/tuned_attention.py:20-81).
template <bool PRECISE, int NB, int STAGE = 0>
__global__ __launch_bounds__(kThreads * NB, 2 / NB) void attn_kernel(AttnParams p) {
  static_assert(STAGE == 0 || NB == 1, "staged calls are general calls");
  // LDS ring: K rows of units i (slot i & 1) run two units ahead of use, V
  // rows one unit ahead.  Iteration i reads K slot (i+1)&1 and V slot i&1
  // while the loads of K unit i+2 and V unit i+1 land in the other slots.
  __shared__ alignas(16) uint8_t ring[4 * kBuf];   // K slot 0 | K slot 1 | V slot 0 | V slot 1
  __shared__ int units[kMaxCount + kMaxRepTiles];
  __shared__ uint32_t maskw[16];
  __shared__ float xm[NB][2][64], xl[NB][2][64];
  __shared__ int nunits_s, nexact_s, wcount[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#ifdef SSA_ATTN_STAMPS
  __shared__ unsigned long long stl[4][kAStampRec];
  auto stamp = [&](int slot, unsigned long long v) {
    if (NB == 1 && lane == 0 && slot < kAStampRec) stl[wave & 3][slot] = v;
  };
  auto tick = [&](int slot) { stamp(slot, __builtin_amdgcn_s_memtime()); };
#endif
  ATTN_TICK(0);
  const int grp = wave >> 2, pair = (wave >> 1) & 1, qw = wave & 1;
  const int TB = p.T / NB;
  // whole tiles first (XCD-grouped), then the pieces of the split tiles
  int work, piece = 0, nparts = 1;
  if (STAGE != 0) {
    work = xcd_remap(blockIdx.x, p.split_from);
    piece = STAGE - 1;
    nparts = 2;
  } else if ((int)blockIdx.x < p.split_from) {
    work = xcd_remap(blockIdx.x, p.split_from);
  } else {
    const int b = blockIdx.x - p.split_from;
    work = p.split_from + b / p.split_k;
    piece = b % p.split_k;
    nparts = p.split_k;
  }
  const int h = work / TB, t = (work % TB) * NB + grp;
  // the table entries first: the unit list waits for them alone, not for
  // the query rows requested after them
  const int first = NB == 1 ? lut_entry(p, h, t, tid) : -1;
  // query operand: lane's query row, dims 16*st + 8*hh + [0,8); its latency
  // overlaps the unit list
  const int r = lane & 31, hh = lane >> 5;
  const long long qrow = (long long)(t * 64 + qw * 32 + r);
  u32x4 qop[8];
  const uint16_t* qp = p.q + qrow * p.q_tok + (long long)h * p.q_head + 8 * hh;
#pragma unroll
  for (int st = 0; st < 8; ++st) qop[st] = ldg16(qp + 16 * st);
  if (NB == 1) {
    own_units<STAGE>(p, h, t, tid, first, units, maskw, wcount, &nunits_s, &nexact_s);
  } else {
    // every page exact, no rep tiles: units are the pages in order
    for (int i = tid; i < p.P; i += kThreads * NB) units[i] = i;
    if (tid == 0) nunits_s = nexact_s = p.P;
  }
  __syncthreads();
  ATTN_TICK(1);
  const int nunits = __builtin_amdgcn_readfirstlane(nunits_s);
  // the piece state's slot: tile (work - split_from) of the split ones, or
  // every tile in a staged call
  const long long pslot = (long long)(((work - (STAGE ? 0 : p.split_from)) * nparts + piece) * NB + grp) * kPieceFloats;
  if (STAGE != 0 && nunits == 0) {
    // no unit of this stage (a table that selects every page, or lists none
    // in the window): the empty state m = -inf, l = 0, O = 0
    for (int i = tid; i < kPieceFloats; i += kThreads) p.part[pslot + i] = i >= 8192 && i < 8256 ? -INFINITY : 0.0f;
    return;
  }
  // this workgroup's units [ibeg, iend): a piece of the list when split,
  // starting at an even unit (so the slot of every step stays known at
  // compile time).  A piece left empty (a list shorter than the pieces)
  // walks unit ibeg and hands on an empty state instead (m = -inf, l = 0,
  // O = 0).
  const int ibeg = STAGE ? 0 : 2 * (nunits * piece / (2 * nparts));
  const int inext = (STAGE || piece + 1 == nparts) ? nunits : 2 * (nunits * (piece + 1) / (2 * nparts));
  const bool empty = inext <= ibeg;
  const int iend = empty ? ibeg + 1 : inext;
  lds_u8* const kbase = (lds_u8*)ring;
  lds_u8* const vbase = (lds_u8*)ring + 2 * kBuf;
  auto kslot = [&](int slot) { return kbase + slot * kBuf; };
  auto vslot = [&](int slot) { return vbase + slot * kBuf; };

  RunMax<!(PRECISE && NB == 1)> rm;
  f32x16 O[4], C = {};
  float ls = 0.f;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) O[dt] = f32x16{};
  const UnitOffsets page_off = unit_offsets(wave, lane, p.kv_tok, 63, NB, true);
  const RepOffsets rep_off = rep_offsets(wave, lane, NB);
  const UnitSources src = unit_sources(p, h);
  // this lane's detail operand rows (rank r % 8 of its half's 12 pairs) in a
  // rep tile's V slot
  const uint32_t det_off = kDetailOff + ((pair * 2 + hh) * 8 + (r & 7)) * 32;
  const uint32_t klane = k_base(pair, lane), vlane = v_base(pair, lane);
  auto unit = [&](int i) { return __builtin_amdgcn_readfirstlane(units[i]); };
  // prologue: K and V of unit ibeg, K of unit ibeg+1 in flight (unit i in
  // slots i & 1); S of unit ibeg and its max
  issue_rows<NB>(p, src, unit(ibeg), 0, wave, lane, page_off, rep_off, kslot(ibeg & 1));
  issue_rows<NB>(p, src, unit(ibeg), 1, wave, lane, page_off, rep_off, vslot(ibeg & 1));
  issue_rows<NB>(p, src, unit(min(ibeg + 1, iend - 1)), 0, wave, lane, page_off, rep_off, kslot((ibeg + 1) & 1));
  wait_loads();
  __syncthreads();
  f32x16 S0 = s_tile(kslot(ibeg & 1), pair, lane, qop), S1;
  float mloc;
  float bias = unit_max(S0, unit(ibeg), pair, lane, p.scale_log2, mloc);
  update_max(mloc, rm, ls, O, C);
  __syncthreads();   // every wave is done with K slot 0 before unit 2's K lands there
  ATTN_TICK(2);
  // Unit ids run ahead in registers (u0 = unit i); the id of unit i+3 is
  // read from LDS in step i-1, so the read completes at its barrier.
  int u0 = unit(ibeg), u1 = unit(min(ibeg + 1, iend - 1)), u2 = unit(min(ibeg + 2, iend - 1));
  int u3raw = units[min(ibeg + 3, iend - 1)];

  // P.V of exact page i (probabilities of Sc, V slot cur), with S(i+1) from
  // the other K slot and its max.  K: the kind of units i+1 and i+2.
  auto page_body = [&](auto kind, int cur, const f32x16& Sc, f32x16& Sn, float nb) {
    constexpr int K = decltype(kind)::value;
    const lds_u8* kb = kslot(cur ^ 1);
    const lds_u8* vb = vslot(cur);
    uint32_t kl = klane, vl = vlane;
    // the 8 K read addresses stay in registers across units; the general
    // call re-forms its 4 V read addresses each step (the two-block call,
    // with registers to spare, keeps those too: 10 fewer vector
    // instructions per step)
    if (NB == 1) asm volatile("" : "+v"(vl));
    if (PRECISE) {
      // Two-term P.V in three stages of 8 matrix products, each carrying a
      // similar share of the vector work, so that the matrix and vector
      // work of this wave overlap throughout the step: S(i+1) with k step 0
      // of unit i's exponentials and splits, the hi/lo products of k step 0
      // with those of k step 1, the products of k step 1 with the max of
      // unit i+1 and the denominator (the lane's fp32 sum of P, gathered in
      // index order as the exponentials form).
      u32x4 ka[8], va[2][4], pb[2], pl[2];
      float P[16], ps = 0.f;
#pragma unroll
      for (int st = 0; st < 4; ++st) ka[st] = k_read(kb, kl, st);
      __builtin_amdgcn_sched_barrier(0);
      Sn = f32x16{};
      // stage A: the 8 products of S(i+1), each with one exponential of
      // k step 0 of unit i, a split every second product, one operand read
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        Sn = mfma32(ka[st], qop[st], Sn);
        if (NB == 2 && st == 0) issue_rows<NB, K>(p, src, u2, 0, wave, lane, page_off, rep_off, kslot(cur));
        if (NB == 2 && st == 3) issue_rows<NB, K>(p, src, u1, 1, wave, lane, page_off, rep_off, vslot(cur ^ 1));
        if (st < 4)
          ka[st + 4] = k_read(kb, kl, st + 4);
        else
          va[0][st - 4] = v_read(vb, vl, 0, st - 4);
        P[st] = __builtin_amdgcn_exp2f(fmaf(Sc[st], p.scale_log2, nb));
        ps += P[st];
        if (st & 1) {
          const u32x2 hl = split_pair(P[st - 1], P[st]);
          pb[0][st >> 1] = hl[0];
          pl[0][st >> 1] = hl[1];
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // stage B: the 8 P.V products of k step 0 (hi, lo), each pair with two
      // exponentials and the split of k step 1, and its V operand read
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        O[dt] = mfma32(va[0][dt], pb[0], O[dt]);
        va[1][dt] = v_read(vb, vl, 1, dt);
        P[8 + 2 * dt] = __builtin_amdgcn_exp2f(fmaf(Sc[8 + 2 * dt], p.scale_log2, nb));
        P[9 + 2 * dt] = __builtin_amdgcn_exp2f(fmaf(Sc[9 + 2 * dt], p.scale_log2, nb));
        ps += P[8 + 2 * dt];
        ps += P[9 + 2 * dt];
        O[dt] = mfma32(va[0][dt], pl[0], O[dt]);
        const u32x2 hl = split_pair(P[8 + 2 * dt], P[9 + 2 * dt]);
        pb[1][dt] = hl[0];
        pl[1][dt] = hl[1];
        __builtin_amdgcn_sched_barrier(0);
      }
      // stage C: the 8 P.V products of k step 1 with the max of unit i+1
      // and the denominator update
      if (NB == 1) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        O[dt] = mfma32(va[1][dt], pb[1], O[dt]);
        if (dt == 0) bias = unit_max<K>(Sn, u1, pair, lane, p.scale_log2, mloc);
        O[dt] = mfma32(va[1][dt], pl[1], O[dt]);
        if (dt == 1) ls += ps;
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      // One instruction stream that keeps the matrix pipe fed: the 8
      // products of S(i+1) each carry two exponentials of unit i and one
      // operand read 4 products ahead; the P.V products of unit i then
      // carry the max of unit i+1.  Scheduling barriers hold the order.
      u32x4 ka[8], va[2][4], pb[2];
      float P[16], ps = 0.f;
#pragma unroll
      for (int st = 0; st < 4; ++st) ka[st] = k_read(kb, kl, st);
      __builtin_amdgcn_sched_barrier(0);
      Sn = f32x16{};
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        Sn = mfma32(ka[st], qop[st], Sn);
        if (NB == 2 && st == 0) issue_rows<NB, K>(p, src, u2, 0, wave, lane, page_off, rep_off, kslot(cur));
        if (NB == 2 && st == 3) issue_rows<NB, K>(p, src, u1, 1, wave, lane, page_off, rep_off, vslot(cur ^ 1));
        if (st < 4)
          ka[st + 4] = k_read(kb, kl, st + 4);
        else
          va[0][st - 4] = v_read(vb, vl, 0, st - 4);
        P[2 * st] = __builtin_amdgcn_exp2f(fmaf(Sc[2 * st], p.scale_log2, nb));
        P[2 * st + 1] = __builtin_amdgcn_exp2f(fmaf(Sc[2 * st + 1], p.scale_log2, nb));
        ps += P[2 * st];
        ps += P[2 * st + 1];
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int o = 8 * ks;
        pb[ks] = u32x4{pack_bf16(P[o + 0], P[o + 1]), pack_bf16(P[o + 2], P[o + 3]), pack_bf16(P[o + 4], P[o + 5]),
                       pack_bf16(P[o + 6], P[o + 7])};
      }
      __builtin_amdgcn_sched_barrier(0);
      // the P.V products, the next max and the running-max update run at
      // raised wave priority: this wave then wins the SIMD's issue slots over
      // the other workgroup's wave in its exponentials or load issue, and the
      // step reaches its barrier sooner (general call only; measured ~6%)
      if (NB == 1) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        O[dt] = mfma32(va[0][dt], pb[0], O[dt]);
        va[1][dt] = v_read(vb, vl, 1, dt);
        if (dt == 1) ls += ps;
        __builtin_amdgcn_sched_barrier(0);
      }
      bias = unit_max<K>(Sn, u1, pair, lane, p.scale_log2, mloc);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) O[dt] = mfma32(va[1][dt], pb[1], O[dt]);
    }
  };

  // The compensation of rep tile i (probabilities of Sc); with NEXT also
  // S(i+1) from the other K slot and its max.  Lane (query r, half hh) holds
  // the 4 reps of pair-local page 2 jp + hh in Sc[4 jp .. 4 jp + 3] (jp =
  // 0..3).
  //  * contrasts: C += D^T B^T; in k = 8 hh + j the products take bf16
  //    weights of lane half hh's 12 (page, contrast) pairs v = 3 jp + a
  //    against A rows = detail[page][a][rank] (the operand tile, whose two
  //    chunks hold v = 0..7 and v = 8..11, 0..3).  Single-term path: 2
  //    products, weights 0..7 and 8..11 (then zeros).  Two-term path (the
  //    reference's _av(c_a, detail_a) on hi + lo parts): 3 products, hi
  //    0..7; hi 8..11 with lo 0..3; lo 4..11 against the words of v = 4..11;
  //  * means: O^T += M^T A^T, one product per dim tile over the pair's 8
  //    pages, k = 8 hh + e holding page e < 4 ? 2 e : 2 e - 7, the lo parts
  //    of its mean weight in half 0 and the hi parts in half 1 (two-term
  //    path; one bf16 term, lo = 0, in the single-term path); M^T is read as
  //    the V operand of k step 0 from the mean rows the loads placed.
  auto rep_body = [&](auto next_c, auto kind, int cur, const f32x16& Sc, f32x16& Sn, float nb) {
    constexpr bool NEXT = decltype(next_c)::value;
    constexpr int K = decltype(kind)::value;
    const lds_u8* kb = kslot(cur ^ 1);
    const lds_u8* vb = vslot(cur);
    uint32_t kl = klane, vl = vlane, dl = det_off;
    if (PRECISE)
      asm volatile("" : "+v"(vl), "+v"(dl));
    else
      asm volatile("" : "+v"(kl), "+v"(vl), "+v"(dl));
    u32x4 ka[8], va[4], dop[2];
    float hw[16];   // probabilities, then at 4 jp the Haar view of page jp
    if constexpr (NEXT) {
#pragma unroll
      for (int st = 0; st < 4; ++st) ka[st] = k_read(kb, kl, st);
      __builtin_amdgcn_sched_barrier(0);
      Sn = f32x16{};
    }
    // the products of S(i+1), each with two exponentials; every second one
    // completes a page and its Haar view
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      if constexpr (NEXT) {
        Sn = mfma32(ka[st], qop[st], Sn);
        if (st < 4) ka[st + 4] = k_read(kb, kl, st + 4);
      }
      if (st >= 4 && st < 6) dop[st - 4] = *(lds_u32x4*)(vb + dl + 16 * (st - 4));
      hw[2 * st] = __builtin_amdgcn_exp2f(fmaf(Sc[2 * st], p.scale_log2, nb));
      hw[2 * st + 1] = __builtin_amdgcn_exp2f(fmaf(Sc[2 * st + 1], p.scale_log2, nb));
      if (st & 1) haar4(hw + 4 * (st >> 1), hw + 4 * (st >> 1));
      __builtin_amdgcn_sched_barrier(0);
    }
    // the contrast products, each with its weights' packing and the reads of
    // mean operands
    auto bw = [&](int v) { return hw[4 * (v / 3) + 1 + v % 3]; };
    auto wsplit = [&](float a, float b) { return PRECISE ? split_pair(a, b) : u32x2{pack_bf16(a, b), 0u}; };
    if constexpr (PRECISE) {
      u32x2 cw[6];   // hi | lo words of the weights v = 2k, 2k + 1
#pragma unroll
      for (int k = 0; k < 4; ++k) cw[k] = split_pair(bw(2 * k), bw(2 * k + 1));
      const u32x4 b0 = {cw[0][0], cw[1][0], cw[2][0], cw[3][0]};
      C = mfma32(dop[0], b0, C);
      cw[4] = split_pair(bw(8), bw(9));
      cw[5] = split_pair(bw(10), bw(11));
      va[0] = v_read(vb, vl, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      const u32x4 b1 = {cw[4][0], cw[5][0], cw[0][1], cw[1][1]};
      C = mfma32(dop[1], b1, C);
      va[1] = v_read(vb, vl, 0, 1);
      va[2] = v_read(vb, vl, 0, 2);
      __builtin_amdgcn_sched_barrier(0);
      const u32x4 a2 = {dop[0][2], dop[0][3], dop[1][0], dop[1][1]};
      const u32x4 b2 = {cw[2][1], cw[3][1], cw[4][1], cw[5][1]};
      C = mfma32(a2, b2, C);
      va[3] = v_read(vb, vl, 0, 3);
      __builtin_amdgcn_sched_barrier(0);
    } else {
      const u32x4 b0 = {pack_bf16(bw(0), bw(1)), pack_bf16(bw(2), bw(3)), pack_bf16(bw(4), bw(5)),
                        pack_bf16(bw(6), bw(7))};
      C = mfma32(dop[0], b0, C);
      va[0] = v_read(vb, vl, 0, 0);
      va[1] = v_read(vb, vl, 0, 1);
      __builtin_amdgcn_sched_barrier(0);
      const u32x4 b1 = {pack_bf16(bw(8), bw(9)), pack_bf16(bw(10), bw(11)), 0u, 0u};
      C = mfma32(dop[1], b1, C);
      va[2] = v_read(vb, vl, 0, 2);
      va[3] = v_read(vb, vl, 0, 3);
      __builtin_amdgcn_sched_barrier(0);
    }
    const u32x2 a01 = wsplit(hw[0], hw[4]), a23 = wsplit(hw[8], hw[12]);
    const u32x2 x0 = halves(a01[1], a01[0]), x1 = halves(a23[1], a23[0]);
    const u32x4 am = {x0[0], x1[0], x0[1], x1[1]};
    if (NEXT && NB == 1) __builtin_amdgcn_s_setprio(1);
    // the mean products with the max of unit i+1 and the denominator
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      O[dt] = mfma32(va[dt], am, O[dt]);
      if constexpr (NEXT) {
        if (dt == 0) bias = unit_max<K>(Sn, u1, pair, lane, p.scale_log2, mloc);
      }
      if (dt == 1) ls += (hw[0] + hw[4]) + (hw[8] + hw[12]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // One unit with a successor: loads of K unit i+2 (clamped to the last
  // unit; a surplus load lands in a slot nobody reads again) and V unit i+1,
  // S of unit i+1, the P.V (or compensation) of unit i, the max of unit i+1
  // (before the last products, so it does not wait behind them in the matrix
  // pipe).  KP: the kind of unit i (page or rep tile); K: that of units
  // i+1 and i+2.
  auto step = [&](auto pvkind, auto kind, auto parity, int i, f32x16& Sc, f32x16& Sn) {
    constexpr int KP = decltype(pvkind)::value;
    constexpr int K = decltype(kind)::value;
    constexpr int cur = decltype(parity)::value;   // i & 1: every paired loop keeps i even
    const int u3 = __builtin_amdgcn_readfirstlane(u3raw);
    ATTN_TICK(8 + 3 * (i - ibeg));
    // the general call issues its loads first; the two-block call (8 waves,
    // half the loads each) spreads them over the first products
    if (NB == 1) {
      issue_rows<NB, K>(p, src, u2, 0, wave, lane, page_off, rep_off, kslot(cur));
      issue_rows<NB, K>(p, src, u1, 1, wave, lane, page_off, rep_off, vslot(cur ^ 1));
    }
    const float nb = bias + rm.neg();
    if constexpr (NB == 1 && KP == 1)
      rep_body(std::true_type{}, kind, cur, Sc, Sn, nb);
    else
      page_body(kind, cur, Sc, Sn, nb);
    update_max(mloc, rm, ls, O, C);
    if (NB == 1) __builtin_amdgcn_s_setprio(0);
    ATTN_TICK(9 + 3 * (i - ibeg));
    u0 = u1;
    u1 = u2;
    u2 = u3;
    u3raw = units[min(i + 4, iend - 1)];
    wait_loads();
    ATTN_TICK(10 + 3 * (i - ibeg));
    __syncthreads();
  };
  // Units are the exact pages, then the rep tiles; every step knows the kind
  // of its units at compile time (i is even in the paired loops, so the
  // parity of npages fixes where the kinds change)
  using PageUnits = std::integral_constant<int, 0>;
  using RepUnits = std::integral_constant<int, 1>;
  using AnyUnits = std::integral_constant<int, 2>;
  using Even = std::integral_constant<int, 0>;
  using Odd = std::integral_constant<int, 1>;
  const int npages = nexact_s;
  int i = ibeg;
  for (; i + 2 < iend && i + 3 < npages; i += 2) {
    step(PageUnits{}, PageUnits{}, Even{}, i, S0, S1);
    step(PageUnits{}, PageUnits{}, Odd{}, i + 1, S1, S0);
  }
  for (; i + 2 < iend && i + 1 < npages; i += 2) {
    step(PageUnits{}, AnyUnits{}, Even{}, i, S0, S1);
    step(PageUnits{}, AnyUnits{}, Odd{}, i + 1, S1, S0);
  }
  if constexpr (NB == 1) {
    // here unit i+1 is a rep tile; unit i is the last page when npages is odd
    if (i + 2 < iend && i < npages) {
      step(PageUnits{}, RepUnits{}, Even{}, i, S0, S1);
      step(RepUnits{}, RepUnits{}, Odd{}, i + 1, S1, S0);
      i += 2;
    }
    for (; i + 2 < iend; i += 2) {
      step(RepUnits{}, RepUnits{}, Even{}, i, S0, S1);
      step(RepUnits{}, RepUnits{}, Odd{}, i + 1, S1, S0);
    }
  }
  ATTN_TICK(3);
  ATTN_STAMP(6, (unsigned long long)npages | (unsigned long long)nunits << 16 | (unsigned long long)ibeg << 32 |
               (unsigned long long)i << 48);
  // one unit with a successor left (units i and i+1 = iend - 1): the same
  // work without the interleaving, each kind chosen at run time
  auto unit_pv = [&](int cur, const f32x16& Sc, float nb) {
    bool rep = false;
    if constexpr (NB == 1) rep = u0 < 0;
    if (rep) {
      f32x16 unused;
      if constexpr (NB == 1) rep_body(std::false_type{}, AnyUnits{}, cur, Sc, unused, nb);
    } else {
      u32x4 pb[2], pl[2];
      probabilities<PRECISE>(Sc, nb, p.scale_log2, pb, pl, ls);
      pv<PRECISE>(pb, pl, vslot(cur), pair, lane, O);
    }
  };
  if (i + 1 < iend) {
    issue_rows<NB>(p, src, u1, 1, wave, lane, page_off, rep_off, vslot((i + 1) & 1));
    S1 = s_tile(kslot((i + 1) & 1), pair, lane, qop);
    unit_pv(i & 1, S0, bias + rm.neg());
    bias = unit_max(S1, u1, pair, lane, p.scale_log2, mloc);
    update_max(mloc, rm, ls, O, C);
    u0 = u1;
    wait_loads();
    __syncthreads();
    ++i;
    S0 = S1;
  }
  // last unit
  {
    u32x4 bop[4];
    if constexpr (NB == 1) {
      // basis rows of dims 32 dt + r (ranks 0..7), for the code accumulator
      const uint16_t* bp = p.basis + ((long long)h * kHeadDim + r) * 8;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) bop[dt] = ldg16(bp + 256 * dt);
    }
    unit_pv(i & 1, S0, bias + rm.neg());
    if constexpr (NB == 1) {
      // O^T += basis . C^T: the two-term operand of C holds the lo parts of
      // ranks 0..7 in k 0..7 and the hi parts in k 8..15
      const u32x2 c01 = split_pair(C[0], C[1]), c23 = split_pair(C[2], C[3]);
      const u32x2 y0 = halves(c01[1], c01[0]), y1 = halves(c23[1], c23[0]);
      const u32x4 cb = {y0[0], y1[0], y0[1], y1[1]};
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) O[dt] = mfma32(bop[dt], cb, O[dt]);
    }
  }
  ATTN_TICK(4);
  __syncthreads();
  // merge the two key halves: pair 1 hands (m, l, O) to pair 0 through LDS.
  // Lanes l and l ^ 32 hold the fp32 partial sums of one query's two 16-key
  // halves (ls).
  float l = 0.0f;
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ls), __float_as_uint(ls), false, false);
    l += __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  // [group][qw][64 items][64 lanes] fp32 = 32 KB per group
  float* xo = reinterpret_cast<float*>(ring) + grp * 8192;
  if (pair == 1) {
    float* d = xo + qw * 4096 + lane;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) d[(16 * dt + i) * 64] = O[dt][i];
    xm[grp][qw][lane] = rm.m;
    xl[grp][qw][lane] = l;
  }
  __syncthreads();
#ifdef SSA_ATTN_STAMPS
  tick(5);
  stamp(7, (unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 4) |
               (unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 20) << 32);
  if (NB == 1 && blockIdx.x < kAStampWGs) {
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's stamp writes
    for (int k = lane; k < kAStampRec; k += 64)
      attn_stamps[((long long)blockIdx.x * 4 + wave) * kAStampRec + k] = stl[wave & 3][k];
  }
#endif
  if (pair == 1) return;
  const float m1 = xm[grp][qw][lane], l1 = xl[grp][qw][lane];
  const float m = rm.m;
  const float mt = fmaxf(m, m1);
  const float mu = mt == -INFINITY ? 0.0f : mt;
  const float a0 = __builtin_amdgcn_exp2f(m - mu), a1 = __builtin_amdgcn_exp2f(m1 - mu);
  const float lt = l * a0 + l1 * a1;
  const float* d = xo + qw * 4096 + lane;
  // the lane's query, dim half and query half, re-formed here so that no
  // register holds them across the unit loop
  int lq = tid;
  asm volatile("" : "+v"(lq));
  const int rq = lq & 31, hq = (lq >> 5) & 1, qq = (lq >> 6) & 1;
  if (nparts > 1) {
    // a piece: its unnormalised state (the two key halves merged) for
    // merge_kernel, in this epilogue's lane layout
    float* slot = p.part + pslot;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x4 po;
#pragma unroll
        for (int c = 0; c < 4; ++c) po[c] = empty ? 0.0f : O[dt][4 * j + c] * a0 + d[(16 * dt + 4 * j + c) * 64] * a1;
        *reinterpret_cast<f32x4*>(slot + ((qq * 16 + dt * 4 + j) * 64 + lq % 64) * 4) = po;
      }
    if (hq == 0) {
      slot[8192 + qq * 32 + rq] = empty ? -INFINITY : mu;
      slot[8256 + qq * 32 + rq] = empty ? 0.0f : lt;
    }
    return;
  }
  const float inv = 1.0f / lt;
  uint16_t* op = p.out + (long long)(t * 64 + qq * 32 + rq) * p.q_tok + (long long)h * p.q_head + 4 * hq;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = (O[dt][4 * j + c] * a0 + d[(16 * dt + 4 * j + c) * 64] * a1) * inv;
      const u32x2 w = {pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3])};
      *reinterpret_cast<u32x2*>(op + 32 * dt + 8 * j) = w;
    }
  }
}

// The split tiles' output: block (s, qw, dh) merges the K pieces of split
// tile s (tile g = s % NB of workgroup split_from + s / NB) for queries
// 32 qw .. 32 qw + 31 and dims 64 dh .. 64 dh + 63 (O = sum_j O_j
// 2^(m_j - M), l likewise, M = max_j m_j, in piece order) and writes
// out = O / l.  Lane l holds the epilogue's lane layout; every load is
// issued before the first use.
template <int K, int NB>
__global__ __launch_bounds__(64) void merge_kernel(const float* part, uint16_t* out, int split_from, int T,
                                                   long long q_tok, long long q_head) {
  const int lane = threadIdx.x, s = blockIdx.x >> 2, qw = (blockIdx.x >> 1) & 1, dh = blockIdx.x & 1;
  const int r = lane & 31, hh = lane >> 5;
  const int TB = T / NB, g = s % NB;
  const int work = split_from + s / NB;
  const int h = work / TB, t = (work % TB) * NB + g;
  float mj[K], lj[K];
  f32x4 v[K][2][4];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const float* sj = part + (long long)(((s / NB) * K + j) * NB + g) * kPieceFloats;
    mj[j] = sj[8192 + qw * 32 + r];
    lj[j] = sj[8256 + qw * 32 + r];
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        v[j][x][jj] = *reinterpret_cast<const f32x4*>(sj + ((qw * 16 + (2 * dh + x) * 4 + jj) * 64 + lane) * 4);
  }
  float M = -INFINITY;
#pragma unroll
  for (int j = 0; j < K; ++j) M = fmaxf(M, mj[j]);
  f32x4 acc[2][4] = {};
  float L = 0.0f;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const float a = __builtin_amdgcn_exp2f(mj[j] - M);
    L += lj[j] * a;
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[x][jj][c] += v[j][x][jj][c] * a;
  }
  const float inv = 1.0f / L;
  uint16_t* op = out + (long long)(t * 64 + qw * 32 + r) * q_tok + (long long)h * q_head + 4 * hh;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const u32x2 w = {pack_bf16(acc[x][jj][0] * inv, acc[x][jj][1] * inv),
                       pack_bf16(acc[x][jj][2] * inv, acc[x][jj][3] * inv)};
      *reinterpret_cast<u32x2*>(op + 32 * (2 * dh + x) + 8 * jj) = w;
    }
}

// Detail operand tiles of one head per block row: rops[h, rt] for the
// ceil(P/16) tiles of the window (96 chunks of 16 bytes each).
__global__ __launch_bounds__(kRepOpChunks) void rep_operands_kernel(const uint16_t* detail, uint16_t* rops, int P,
                                                                   int HP, int RT) {
  const int rt = blockIdx.x, h = blockIdx.y, c = threadIdx.x;
  const u32x4 w = rep_operand_chunk(detail + (long long)h * HP * 24, P, rt, c);
  *reinterpret_cast<u32x4*>(rops + ((long long)h * RT + rt) * (kRepOpBytes / 2) + 8 * c) = w;
}

// Compute units of the current device (cached per device).
int device_cus(int* out) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cus[kMaxDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return (int)e;
    n = n > 0 ? n : 1;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  *out = n;
  return (int)hipSuccess;
}

// The split a call runs: the workgroups past the last multiple of the CU
// count run as pieces, so the last round spreads over every CU.  The
// general call (NB = 1, two workgroups per CU) splits them in 2; the
// two-block call (NB = 2, one per CU) in 4.  Returns the number of split
// workgroups (0: none), the pieces per workgroup and the workspace bytes.
int split_plan(int wgs, int nb, int* split_wgs, int* k, long long* bytes) {
  int cus = 0;
  const int e = device_cus(&cus);
  if (e != (int)hipSuccess) return e;
  const int r = wgs % cus;
  *split_wgs = r;
  *k = nb == 1 ? 2 : 4;
  *bytes = (long long)r * *k * nb * kPieceFloats * 4;
  return (int)hipSuccess;
}

// Flag bits of ssa_attention.
constexpr int kTwoTerm = 1, kDense = 2, kStaged = 4;

// Whether a call runs the two-block dense kernel: the caller's flag, a table
// of every page and an even number of query blocks.
bool dense_call(int flags, int count, int pages, int n_tokens) {
  return (flags & kDense) && count == pages && (n_tokens / 64) % 2 == 0;
}

// Workspace bytes of a staged call: two piece states per tile.
long long staged_bytes(int wgs) { return (long long)wgs * 2 * kPieceFloats * 4; }

}  // namespace

extern "C" {

// Step stamps of the last one-block attention launch in a measurement build:
// copies [kAStampWGs, 4 waves, kAStampRec] uint64 into `out` (host memory,
// `bytes` >= its size) and returns 0; hipErrorNotSupported in the product
// library.
int ssa_attn_stamps(void* out, long long bytes) {
#ifdef SSA_ATTN_STAMPS
  if (out == nullptr || bytes < (long long)sizeof(attn_stamps)) return (int)hipErrorInvalidValue;
  return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(attn_stamps), sizeof(attn_stamps));
#else
  (void)out;
  (void)bytes;
  return (int)hipErrorNotSupported;
#endif
}

long long ssa_attention_workspace_bytes(int n_tokens, int heads, int pages, int count, int flags) {
  if (n_tokens <= 0 || n_tokens % 64 || heads <= 0 || pages <= 0 || count <= 0 || count > pages) return -1;
  if ((flags & kStaged) && (flags & kDense)) return -1;
  if (flags & kStaged) return staged_bytes(heads * (n_tokens / 64));
  const int nb = dense_call(flags, count, pages, n_tokens) ? 2 : 1;
  int r = 0, k = 1;
  long long bytes = 0;
  if (split_plan(heads * (n_tokens / 64) / nb, nb, &r, &k, &bytes) != (int)hipSuccess) return -1;
  return bytes;
}

int ssa_rep_operands(const void* detail, void* rep_ops, int heads, int pages, int head_pages, int rep_tiles,
                     hipStream_t stream) {
  if (heads <= 0 || pages <= 0 || pages > 512 || head_pages < pages || rep_tiles < (pages + 15) / 16 || !detail ||
      !rep_ops || ((uintptr_t)rep_ops & 15))
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(rep_operands_kernel, dim3((pages + 15) / 16, heads), dim3(kRepOpChunks), 0, stream,
                     (const uint16_t*)detail, (uint16_t*)rep_ops, pages, head_pages, rep_tiles);
  return (int)hipGetLastError();
}

int ssa_attention(const void* q, const void* k, const void* v, const void* keys, const void* mean, const void* basis,
                  const void* rep_ops, const int32_t* ids, void* out, int n_tokens, int heads, int pages,
                  int head_pages, int rep_tiles, int count, long long kv_token_stride, long long kv_head_stride,
                  int flags, void* workspace, long long workspace_bytes, hipStream_t stream) {
  if (n_tokens <= 0 || n_tokens % 64 || heads <= 0 || pages <= 0 || pages > 512 || count <= 0 ||
      count > kMaxCount || count > pages || head_pages < pages)
    return (int)hipErrorInvalidValue;
  const bool dense = dense_call(flags, count, pages, n_tokens);
  const bool staged = (flags & kStaged) != 0;
  // a staged call is a general call that needs the workspace for its states
  if (staged && ((flags & kDense) || !workspace || workspace_bytes < staged_bytes(heads * (n_tokens / 64)) ||
                 ((uintptr_t)workspace & 15)))
    return (int)hipErrorInvalidValue;
  // the general call reads page means, the basis and the operand tiles (in
  // 16-byte rows)
  if (!dense && (rep_tiles < (pages + 15) / 16 || !mean || !basis || !rep_ops ||
                 (((uintptr_t)mean | (uintptr_t)basis | (uintptr_t)rep_ops) & 15)))
    return (int)hipErrorInvalidValue;
  // a K/V row is 128 elements; page byte offsets of the window fit 32 bits
  if (kv_token_stride < kHeadDim || kv_head_stride < 0 || 128.0 * (double)kv_token_stride * pages >= 4294967296.0)
    return (int)hipErrorInvalidValue;
  AttnParams p;
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.rk = (const uint16_t*)keys;
  p.mean = (const uint16_t*)mean;
  p.basis = (const uint16_t*)basis;
  p.rops = (const uint16_t*)rep_ops;
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
  p.RT = rep_tiles;
  p.C = count;
  p.scale_log2 = kLog2e / sqrtf((float)kHeadDim);
  // a call whose caller states that every LUT row lists each page once
  // (flags bit 1: a dense call) runs, with an even number of blocks, two
  // blocks per workgroup on one shared K/V stream of pages 0..P-1; ids,
  // page means, basis and operand tiles are then not read.  Without the
  // flag the LUT is walked as given.
  const int nb = dense ? 2 : 1;
  const int wgs = heads * p.T / nb;
  p.part = nullptr;
  p.split_from = wgs;
  p.split_k = 1;
  // with a workspace of ssa_attention_workspace_bytes, the workgroups past
  // the last multiple of the CU count run as pieces, merged by merge_kernel
  int r = 0, pieces = 1;
  long long need = 0;
  const int e = split_plan(wgs, nb, &r, &pieces, &need);
  if (e != (int)hipSuccess) return e;
  if (staged) {
    // the exact pages of every tile, then the rep tiles of every tile, each
    // launch leaving per-tile states; merge_kernel combines the two
    p.part = (float*)workspace;
    if (flags & kTwoTerm) {
      hipLaunchKernelGGL((attn_kernel<true, 1, 1>), dim3(wgs), dim3(kThreads), 0, stream, p);
      hipLaunchKernelGGL((attn_kernel<true, 1, 2>), dim3(wgs), dim3(kThreads), 0, stream, p);
    } else {
      hipLaunchKernelGGL((attn_kernel<false, 1, 1>), dim3(wgs), dim3(kThreads), 0, stream, p);
      hipLaunchKernelGGL((attn_kernel<false, 1, 2>), dim3(wgs), dim3(kThreads), 0, stream, p);
    }
    hipLaunchKernelGGL((merge_kernel<2, 1>), dim3(4 * wgs), dim3(64), 0, stream, p.part, p.out, 0, p.T, p.q_tok,
                       p.q_head);
    return (int)hipGetLastError();
  }
  if (r > 0 && workspace && workspace_bytes >= need && ((uintptr_t)workspace & 15) == 0) {
    p.part = (float*)workspace;
    p.split_from = wgs - r;
    p.split_k = pieces;
  }
  const dim3 grid(p.split_from + (wgs - p.split_from) * p.split_k);
  if (dense) {
    if (flags & kTwoTerm)
      hipLaunchKernelGGL((attn_kernel<true, 2>), grid, dim3(2 * kThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((attn_kernel<false, 2>), grid, dim3(2 * kThreads), 0, stream, p);
    if (p.split_k > 1)
      hipLaunchKernelGGL((merge_kernel<4, 2>), dim3(4 * 2 * (wgs - p.split_from)), dim3(64), 0, stream, p.part,
                         p.out, p.split_from, p.T, p.q_tok, p.q_head);
  } else {
    if (flags & kTwoTerm)
      hipLaunchKernelGGL((attn_kernel<true, 1>), grid, dim3(kThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((attn_kernel<false, 1>), grid, dim3(kThreads), 0, stream, p);
    if (p.split_k > 1)
      hipLaunchKernelGGL((merge_kernel<2, 1>), dim3(4 * (wgs - p.split_from)), dim3(64), 0, stream, p.part,
                         p.out, p.split_from, p.T, p.q_tok, p.q_head);
  }
  return (int)hipGetLastError();
}

}  // extern "C"
