// Shared device helpers for the gfx950 page-sparse attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ssa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kHeadDim = 128;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float bf16_to_f32(uint32_t raw16) { return __uint_as_float(raw16 << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even pack of two floats (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  bf16x2 r;
  r[0] = (__bf16)lo;
  r[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint16_t to_bf16(float x) { return (uint16_t)(pack_bf16(x, 0.f) & 0xffffu); }

__device__ __forceinline__ u32x4 ldg16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// D[32x32] += A[32x16] * B[16x32], bf16 inputs, fp32 accumulate.
// Lane l: A row l%32, k = 8*(l/32)+i; B col l%32, same k; D col l%32,
// rows 8*(i/4) + 4*(l/32) + i%4 for accumulator item i.
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 c, 0, 0, 0);
}

// Row of probe m (0..15) in its 64-query block: round(63 m / 15), the 16
// evenly spaced rows of VR/runtime.py:84 (linspace(0, 63, 16).round()).
__device__ __forceinline__ int probe_row(int m) { return (42 * m + 5) / 10; }

// Monotone map of a float to an unsigned key (larger float -> larger key);
// -0.0 and +0.0 share a key so equal floats compare equal.
__device__ __forceinline__ uint32_t orderable(float f) {
  if (f == 0.0f) f = 0.0f;
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Flattened block id -> work item, keeping contiguous work ranges on one XCD
// (the dispatcher round-robins consecutive workgroups over the 8 XCDs).
__device__ __forceinline__ int xcd_remap(int b, int total) {
  if (total % 8 != 0) return b;
  return (b % 8) * (total / 8) + b / 8;
}

// s_waitcnt vmcnt(0) (expcnt/lgkmcnt left at their maxima) as the intrinsic,
// so the compiler's own wait-count tracking sees it.
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// 16-byte global->LDS load of one wave: lane l's 16 bytes at base + off
// (bytes; base wave-uniform in SGPRs, off per lane) land at lds + 16*l.
// The LDS base goes in through the "{m0}" operand, so the compiler writes
// M0 itself and knows its value (the asm reads M0 and clobbers nothing);
// the s_nop keeps the one wait state an M0 write needs before an LDS DMA.
// Issued from inline asm so the compiler does not fence later LDS reads on
// it; wait_loads() (and a barrier, for other waves' loads) orders it.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

// N consecutive 1 KB global->LDS loads of one wave: load jj reads base +
// off[jj] + jj * 1024 (per lane) into lds + jj * 1024 + 16 * lane, with one
// M0 value for all of them.
template <int N>
__device__ __forceinline__ void dma_rows(const void* base, const uint32_t (&off)[4], uint32_t lds) {
  if constexpr (N == 4) {
    asm volatile(
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %4\n\t"
        "global_load_lds_dwordx4 %1, %4 offset:1024\n\t"
        "global_load_lds_dwordx4 %2, %4 offset:2048\n\t"
        "global_load_lds_dwordx4 %3, %4 offset:3072" ::"v"(off[0]),
        "v"(off[1]), "v"(off[2]), "v"(off[3]), "s"(base), "{m0}"(lds)
        : "memory");
  } else {
    static_assert(N == 2, "2 or 4 loads");
    asm volatile(
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %2\n\t"
        "global_load_lds_dwordx4 %1, %2 offset:1024" ::"v"(off[0]),
        "v"(off[1]), "s"(base), "{m0}"(lds)
        : "memory");
  }
}

// Lane l's partner l ^ O (O = 32, 16, 8, 4, 2, 1) without the LDS
// crossbar: the lane-half and row-pair swaps return both lanes of a pair, a
// row rotation by 8 and the quad permutations are exact partners, and the
// swizzle's xor mode covers 4.  Same values as __shfl_xor(v, O).
__device__ __forceinline__ uint32_t lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

template <int O>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
  if constexpr (O == 32) {
    const auto s = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane_id() & 32) ? s[0] : s[1];
  } else if constexpr (O == 16) {
    const auto s = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane_id() & 16) ? s[0] : s[1];
  } else if constexpr (O == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);   // row_ror:8
  } else if constexpr (O == 4) {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x101F);                       // xor 4 in 32 lanes
  } else if constexpr (O == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);    // quad_perm 2,3,0,1
  } else {
    static_assert(O == 1, "xor offsets 32, 16, 8, 4, 2, 1");
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);    // quad_perm 1,0,3,2
  }
}

template <int O>
__device__ __forceinline__ float xor_lane(float v) {
  return __uint_as_float(xor_lane<O>(__float_as_uint(v)));
}

template <int O>
__device__ __forceinline__ int xor_lane(int v) {
  return (int)xor_lane<O>((uint32_t)v);
}

template <int O>
__device__ __forceinline__ double xor_lane(double v) {
  const unsigned long long u = (unsigned long long)__double_as_longlong(v);
  const uint32_t lo = xor_lane<O>((uint32_t)u), hi = xor_lane<O>((uint32_t)(u >> 32));
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Butterfly over the wave (steps 32, 16, 8, 4, 2, 1) with a commutative op:
// every lane ends with the reduction, bit for bit as over __shfl_xor.  The
// swaps hand both lanes of a pair to op; for steps 8 .. 1 a rotation of the
// 16-lane row reaches a lane that, after the larger steps, holds the value
// of lane l ^ o (the values agree across the offsets already combined).
template <int CTRL, typename T>
__device__ __forceinline__ T rotate_row(T v) {
  if constexpr (sizeof(T) == 8) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
  } else {
    return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
  }
}

template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
  if constexpr (sizeof(T) == 8) {
    v = op(v, xor_lane<32>(v));
    v = op(v, xor_lane<16>(v));
  } else {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto s32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = op(__builtin_bit_cast(T, (uint32_t)s32[0]), __builtin_bit_cast(T, (uint32_t)s32[1]));
    const uint32_t w = __builtin_bit_cast(uint32_t, v);
    const auto s16 = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    v = op(__builtin_bit_cast(T, (uint32_t)s16[0]), __builtin_bit_cast(T, (uint32_t)s16[1]));
  }
  v = op(v, rotate_row<0x128>(v));   // row_ror:8
  v = op(v, rotate_row<0x124>(v));   // row_ror:4
  v = op(v, rotate_row<0x122>(v));   // row_ror:2
  v = op(v, rotate_row<0x121>(v));   // row_ror:1
  return v;
}

// Detail operand tiles of the compensation.  A rep tile covers pages
// 16 rt .. 16 rt + 15 of the window; its operand tile (kRepOpBytes) holds, for
// each (pair, hh, rank) = the matrix-pipe A rows of one lane, the rank-`rank`
// element of detail[page][a] for the 12 (page, contrast) pairs that lane half
// hh of key pair `pair` weighs: v = 3 jp + a, page 16 rt + 8 pair + 2 jp + hh
// (jp = 0..3, a = 0..2), as two 16-byte chunks c = ((pair * 2 + hh) * 8 +
// rank) * 2 + m, element j -> v = (8 m + j) mod 12: chunk 0 holds v = 0..7,
// chunk 1 v = 8..11 then 0..3.  These are the A operands of the contrast
// products: with one bf16 term per weight, chunk 0 against weights 0..7 and
// chunk 1 against weights 8..11 (zeros against its second half); with two
// terms (hi + lo parts), chunk 0 against hi 0..7, chunk 1 against hi 8..11
// and lo 0..3, and the words of v = 4..11 (second half of chunk 0, first half
// of chunk 1) against lo 4..11.  Pages >= P read zero.
constexpr int kRepOpBytes = 1024;
constexpr int kRepOpChunks = kRepOpBytes / 16;

// Chunk c of operand tile rt from one head's detail rows [HP, 3, 8] bf16.
// Shared by every kernel that writes the tiles, so they agree bit for bit.
__device__ __forceinline__ u32x4 rep_operand_chunk(const uint16_t* det, int P, int rt, int c) {
  const int m = c & 1, rank = (c >> 1) & 7, hh = (c >> 4) & 1, pair = c >> 5;
  u32x4 out;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    uint32_t packed = 0;
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int v = (8 * m + 2 * x + y) % 12, jp = v / 3, a = v % 3;
      const int pg = 16 * rt + 8 * pair + 2 * jp + hh;
      const uint32_t val = pg < P ? (uint32_t)det[pg * 24 + a * 8 + rank] : 0u;
      packed |= val << (16 * y);
    }
    out[x] = packed;
  }
  return out;
}

}  // namespace ssa
