// Device helpers shared by the gfx950 kernels: bf16/fp16 conversions, packed bf16 dot products and wave-level
// reductions. Wavefronts are 64 lanes wide on CDNA; every reduction here assumes that.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bp {

// Weight kinds of the skinny kernels.
constexpr int kBf16 = 0;
constexpr int kInt8 = 1;

constexpr int kWave = 64;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// bf16 -> fp32 is exact: the bf16 bits are the top half of the fp32 pattern.
__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// fp32 -> bf16 bits, round to nearest even (what torch's .to(torch.bfloat16) does); NaN stays NaN.
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float round_to_bf16(float f) { return bf16_bits_to_float(float_to_bf16_bits(f)); }
__device__ __forceinline__ float round_to_f16(float f) { return static_cast<float>(static_cast<_Float16>(f)); }

// acc + a.lo * b.lo + a.hi * b.hi with a, b two packed bf16 values (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc, false);
}

// Two signed bytes of d (at bit offsets sh and sh + 8) as a packed pair of bf16 values; exact for |q| <= 128.
__device__ __forceinline__ uint32_t i8pair_to_bf16x2(uint32_t d, int sh) {
  const float lo = static_cast<float>(static_cast<int8_t>(d >> sh));
  const float hi = static_cast<float>(static_cast<int8_t>(d >> (sh + 8)));
  // bytes 2,3 of lo then bytes 2,3 of hi (v_perm_b32 selector: sources are {hi: bytes 4-7, lo: bytes 0-3})
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// Global-memory views of generic pointers. Pointers read from memory (not kernel arguments) are otherwise
// accessed with flat instructions, which also count against the LDS wait counter, so every LDS access would wait
// for all outstanding memory loads.
template <class T>
using gptr = __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<const T> as_global(const T* p) {
  return (gptr<const T>)(p);
}
template <class T>
__device__ __forceinline__ gptr<T> as_global_mut(T* p) {
  return (gptr<T>)(p);
}

// Whether the byte ranges [a, a + na) and [b, b + nb) intersect (a null pointer is an empty range).
inline bool ranges_overlap(const void* a, int64_t na, const void* b, int64_t nb) {
  if (a == nullptr || b == nullptr || na <= 0 || nb <= 0) return false;
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + static_cast<uintptr_t>(nb) && pb < pa + static_cast<uintptr_t>(na);
}

// A raw buffer resource over `bytes` bytes at p (gfx9 word 3: 32-bit data format, no swizzle, no index stride).
// A load at an offset past `bytes` returns zeros without a memory request.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

// The tile of workgroup b of a row of T: the hardware deals a grid's workgroups to the 8 XCDs in turn (b % 8), and
// this gives each XCD one contiguous run of tiles, so neighbouring tiles that share cache lines (a scale row's 32
// bytes per 16 rows) meet in one XCD's L2 instead of four.
constexpr int kXcds = 8;
__device__ __forceinline__ int64_t xcd_tile(int64_t b, int64_t T) {
  const int64_t x = b % kXcds, q = T / kXcds, r = T % kXcds;
  return x * q + (x < r ? x : r) + b / kXcds;
}

// Load a scale element of the given dtype code as fp32 (0 = bf16, 1 = fp16, 2 = fp32).
__device__ __forceinline__ float load_scale(const void* p, int64_t i, int dt) {
  if (dt == 0) return bf16_bits_to_float(as_global(static_cast<const uint16_t*>(p))[i]);
  if (dt == 1) return static_cast<float>(as_global(static_cast<const _Float16*>(p))[i]);
  return as_global(static_cast<const float*>(p))[i];
}

// Sum of v over the 64 lanes of the wave, for P values at once (P a power of two). Butterfly stages pair lanes
// l and l ^ d for d = 32, 16, ..., 1; while more than one value is left, each stage also halves the values a lane
// keeps (the lane with bit d set keeps the upper half). On return:
//   P >= 64: lane l holds, in v[0 .. P/64), the totals of indices [l * P/64, (l + 1) * P/64);
//   P <  64: v[0] of lane l holds the total of index l / (64 / P) (all 64/P lanes of a group hold the same).
// The addition tree of every index is the same for every P (pairs by lane bit 5, then 4, ..., then 0), so a total
// does not depend on how many other values were reduced with it.
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ float dpp_f32(float x, float old = 0.0f) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(x), CTRL, ROW_MASK, BANK_MASK, false));
}

// One stage pairs, for j < P/2, lane l's v[j] (bit d of l clear) or v[j + P/2] (bit d set) with the same index at
// lane l ^ d. Every exchange stays in the VALU: d = 32 and d = 16 are one v_permlane{32,16}_swap per pair (the swap
// leaves lane l's kept value in one register and its partner's in the other), d = 8 is a row rotation by 8, d = 4
// a row shift by 4 in each direction under bank masks (lanes with bit 2 clear are banks 0 and 2 of their row),
// d = 2 and d = 1 are quad permutations. Each sum is kept + received, as a shuffle would give it.
template <int P, int D>
__device__ __forceinline__ void reduce_stage(float* v, int lane) {
  constexpr int H = P > 1 ? P / 2 : 1;
  const bool hi = (lane & D) != 0;
#pragma unroll
  for (int j = 0; j < H; ++j) {
    const float a = v[j];
    const float b = P > 1 ? v[j + P / 2] : v[j];
    if constexpr (D == 32 || D == 16) {
      const auto r = D == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false)
                             : __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
      v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else if constexpr (D == 4) {
      const float lo_recv = dpp_f32<0x104, 0xF, 0x5>(a);           // row_shl:4 into lanes with bit 2 clear
      const float recv = dpp_f32<0x114, 0xF, 0xA>(b, lo_recv);     // row_shr:4 into lanes with bit 2 set
      v[j] = (hi ? b : a) + recv;
    } else {
      constexpr int ctrl = D == 8 ? 0x128 : D == 2 ? 0x4E : 0xB1;  // row_ror:8, quad_perm [2,3,0,1], [1,0,3,2]
      v[j] = (hi ? b : a) + dpp_f32<ctrl>(hi ? a : b);
    }
  }
}

template <int P>
__device__ __forceinline__ void wave_transpose_reduce(float* v, int lane) {
  static_assert((P & (P - 1)) == 0, "P must be a power of two");
  reduce_stage<P, 32>(v, lane);
  reduce_stage<(P > 2 ? P / 2 : 1), 16>(v, lane);
  reduce_stage<(P > 4 ? P / 4 : 1), 8>(v, lane);
  reduce_stage<(P > 8 ? P / 8 : 1), 4>(v, lane);
  reduce_stage<(P > 16 ? P / 16 : 1), 2>(v, lane);
  reduce_stage<(P > 32 ? P / 32 : 1), 1>(v, lane);
}

// One stage of an xor butterfly without LDS traffic: op(v, v of lane l ^ D) for a commutative op, so every lane
// gets exactly what `op(v, __shfl_xor(v, D))` gives. D = 32, 16: a v_permlane{32,16}_swap of two copies of v
// (one result register holds the lane's own value, the other its partner's); D = 8: row_ror:8; D = 4: row_shl:4
// into the lanes with bit 2 clear and row_shr:4 into the others (bank masks); D = 2, 1: quad permutations.
template <int D, class Op>
__device__ __forceinline__ float xor_stage(float v, Op op) {
  if constexpr (D == 32 || D == 16) {
    const auto r = D == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false)
                           : __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  } else if constexpr (D == 4) {
    const float lo_recv = dpp_f32<0x104, 0xF, 0x5>(v);
    return op(v, dpp_f32<0x114, 0xF, 0xA>(v, lo_recv));
  } else {
    static_assert(D == 8 || D == 2 || D == 1, "xor distance");
    return op(v, dpp_f32<D == 8 ? 0x128 : D == 2 ? 0x4E : 0xB1>(v));
  }
}

struct AddOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// Butterfly over the lane bits D_LO .. 32 (D_LO a power of two): the stages of `for (o = D_LO; o < 64; o <<= 1)
// v = op(v, __shfl_xor(v, o))` in that order, and D_LO = 1 in the order 32, 16, ..., 1 when DOWN (the usual
// whole-wave reduction, every lane ends with the total).
template <bool DOWN, int D_LO = 1, class Op>
__device__ __forceinline__ float xor_butterfly(float v, Op op) {
  if constexpr (DOWN) {
    v = xor_stage<32>(v, op);
    v = xor_stage<16>(v, op);
    v = xor_stage<8>(v, op);
    v = xor_stage<4>(v, op);
    v = xor_stage<2>(v, op);
    return xor_stage<1>(v, op);
  } else {
    if constexpr (D_LO <= 1) v = xor_stage<1>(v, op);
    if constexpr (D_LO <= 2) v = xor_stage<2>(v, op);
    if constexpr (D_LO <= 4) v = xor_stage<4>(v, op);
    if constexpr (D_LO <= 8) v = xor_stage<8>(v, op);
    if constexpr (D_LO <= 16) v = xor_stage<16>(v, op);
    return xor_stage<32>(v, op);
  }
}

// Sum of squares of a bf16 row of n elements in LDS (8-byte aligned), in a fixed order that one 64-lane wave
// computes alone: lane l adds, in order, the squares of elements 256 j + 4 l + e (j = 0, 1, ...; e = 0 .. 3;
// elements past n left out), then the lanes are added by a butterfly pairing lane l with lane l ^ d for d = 32,
// 16, ..., 1 (wave_transpose_reduce: permlane swaps and DPP, no LDS round trips). Every lane of every wave that runs
// it gets the same total, so the RMS norms of the decode step (separate or inside a linear's launch) and the
// renormalisations of the linear set agree bit for bit whatever their workgroup shapes. The reads of eight steps
// are issued before their squares are added (the additions stay in order).
__device__ __forceinline__ float wave_sumsq_lds(const uint16_t* row, int n) {
  const int lane = static_cast<int>(threadIdx.x) & 63;
  float s = 0.f;
  int base = 4 * lane;
  for (; base + 7 * 256 + 4 <= n; base += 8 * 256) {
    uint2 q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = *reinterpret_cast<const uint2*>(row + base + 256 * j);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f0 = __uint_as_float(q[j].x << 16), f1 = __uint_as_float(q[j].x & 0xffff0000u);
      const float f2 = __uint_as_float(q[j].y << 16), f3 = __uint_as_float(q[j].y & 0xffff0000u);
      s += f0 * f0;
      s += f1 * f1;
      s += f2 * f2;
      s += f3 * f3;
    }
  }
  for (; base < n; base += 256) {
    if (base + 4 <= n) {
      const uint2 q = *reinterpret_cast<const uint2*>(row + base);
      const float f0 = __uint_as_float(q.x << 16), f1 = __uint_as_float(q.x & 0xffff0000u);
      const float f2 = __uint_as_float(q.y << 16), f3 = __uint_as_float(q.y & 0xffff0000u);
      s += f0 * f0;
      s += f1 * f1;
      s += f2 * f2;
      s += f3 * f3;
    } else {
      for (int e = 0; base + e < n; ++e) {
        const float f = bf16_bits_to_float(row[base + e]);
        s += f * f;
      }
    }
  }
  wave_transpose_reduce<1>(&s, lane);
  return s;
}

// Sum of v over the 64 lanes with DPP moves only (no LDS traffic): pairs within quads, quads within half-rows,
// half-rows within rows of 16 (after which every lane of a row holds the row's sum), then rows 0..3 accumulated
// into row 3 through row broadcasts. The order is fixed, so the result is deterministic; it is returned to every
// lane (the value of lane 63).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f32<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141, 0xF>(v);  // row_half_mirror
  v += dpp_f32<0x140, 0xF>(v);  // row_mirror
  v += dpp_f32<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_f32<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Totals of four rows' per-lane partial sums a0..a3: every row is added in the same order, ((x[j] + x[j + 32]) +
// (x[j + 16] + x[j + 48])) for j < 16 (v_permlane32_swap, then v_permlane16_swap), then a butterfly over 16 lanes;
// returns with a0's total in lanes 0..15, a2's in 16..31, a1's in 32..47 and a3's in 48..63.
__device__ __forceinline__ float wave_sum4_rows(float a0, float a1, float a2, float a3) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a0), __float_as_uint(a1), false, false);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(a2), __float_as_uint(a3), false, false);
  // p: {[a0 lanes 0-31 | a1 lanes 0-31], [a0 lanes 32-63 | a1 lanes 32-63]}, q likewise for a2, a3
  const float b01 = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const float b23 = __uint_as_float(q[0]) + __uint_as_float(q[1]);
  // odd 16-lane rows of b01 <-> even rows of b23: {[b01 r0, b23 r0, b01 r2, b23 r2], [b01 r1, b23 r1, b01 r3, b23 r3]}
  const auto u = __builtin_amdgcn_permlane16_swap(__float_as_uint(b01), __float_as_uint(b23), false, false);
  float c = __uint_as_float(u[0]) + __uint_as_float(u[1]);
  c += dpp_f32<0xB1, 0xF>(c);   // quad_perm [1,0,3,2]
  c += dpp_f32<0x4E, 0xF>(c);   // quad_perm [2,3,0,1]
  c += dpp_f32<0x141, 0xF>(c);  // row_half_mirror
  c += dpp_f32<0x140, 0xF>(c);  // row_mirror
  return c;
}

}  // namespace bp
