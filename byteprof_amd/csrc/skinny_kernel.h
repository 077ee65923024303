// Skinny weight-only matmul kernel template for gfx950: y[M, N] = x[M, K] . W[N, K]^T with up to MT activation
// rows per launch, bf16 activations, fp32 accumulation, bf16 output. Weights are bf16, or int8 with one scale per
// output row (the int8 -> bf16 conversion happens in registers as the weights stream in; the scale multiplies the
// fp32 sum).
//
// Work decomposition (HBM-bound: every weight byte is read exactly once):
//   - a workgroup owns ROWS consecutive weight rows and WAVES wavefronts;
//   - K is cut into chunks of 64 lanes x 16 bytes (512 bf16 or 1024 int8 weights); chunk c of the workgroup's
//     K range goes to wave c % WAVES, so one wave-wide load reads 1 KiB of one row, fully coalesced;
//   - each lane keeps ROWS x MT fp32 partial sums and does 2 products per v_dot2_f32_bf16;
//   - the lane partials are added across the wave by a butterfly that also transposes (wave_transpose_reduce),
//     the wave totals are added in LDS in wave order, and the row's total is scaled / rounded / stored;
//   - with split > 1, grid.y workgroups take consecutive K ranges and store fp32 partials; splitk_reduce adds
//     them in split order.
// The order of every sum depends on (K, WAVES, split) only, so an output row is bitwise independent of M, of
// MT, of ROWS and of which other rows share the launch.
//
// Reference semantics: byteprof/optim/skinny.py:36-90 (kernel and split reduce), :111-166 (launch, skinny_mm);
// byteprof/quant/triton_int8.py:16-47 (one-row int8 product).
#pragma once

#include "common.h"

namespace bp {

// Weight kinds.
constexpr int kBf16 = 0;
constexpr int kInt8 = 1;

template <int KIND>
struct Layout {
  static constexpr int kElemBytes = KIND == kBf16 ? 2 : 1;
  static constexpr int kEpl = 16 / kElemBytes;   // weight elements per lane per chunk (one 16-byte load)
  static constexpr int kChunk = kWave * kEpl;    // elements per chunk
  static constexpr int kXDwords = kEpl / 2;      // packed bf16 activation pairs per lane per chunk
};

using SkinnyFn = void (*)(const uint16_t*, const uint8_t*, const void*, int, uint16_t*, float*, int, int64_t,
                          int64_t, int);

// Loads the 16 weight bytes of one lane (VEC: one aligned 16-byte non-temporal load; otherwise element loads
// with a bound check per element, for K not a multiple of the vector width or unaligned pointers).
template <int KIND, bool VEC>
__device__ __forceinline__ u32x4 load_w(const uint8_t* __restrict__ w, int64_t row, int64_t K, int64_t k0) {
  using L = Layout<KIND>;
  if constexpr (VEC) {
    const u32x4* p = reinterpret_cast<const u32x4*>(w + (row * K + k0) * L::kElemBytes);
    return __builtin_nontemporal_load(p);
  } else {
    uint32_t d[4] = {0u, 0u, 0u, 0u};
    if constexpr (KIND == kBf16) {
      const uint16_t* p = reinterpret_cast<const uint16_t*>(w) + row * K;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (k0 + e < K) d[e >> 1] |= static_cast<uint32_t>(p[k0 + e]) << (16 * (e & 1));
    } else {
      const uint8_t* p = w + row * K;
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (k0 + e < K) d[e >> 2] |= static_cast<uint32_t>(p[k0 + e]) << (8 * (e & 3));
    }
    return u32x4{d[0], d[1], d[2], d[3]};
  }
}

// Loads kEpl activations x[m, k0 .. k0 + kEpl) as packed bf16 pairs (zeros past K).
template <int KIND, bool VEC>
__device__ __forceinline__ void load_x(const uint16_t* __restrict__ xrow, int64_t K, int64_t k0,
                                       uint32_t (&out)[Layout<KIND>::kXDwords]) {
  using L = Layout<KIND>;
  if constexpr (VEC) {
    const u32x4* p = reinterpret_cast<const u32x4*>(xrow + k0);
#pragma unroll
    for (int j = 0; j < L::kXDwords / 4; ++j) {
      const u32x4 t = p[j];
      out[4 * j + 0] = t.x;
      out[4 * j + 1] = t.y;
      out[4 * j + 2] = t.z;
      out[4 * j + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < L::kXDwords; ++j) {
      const uint32_t lo = (k0 + 2 * j < K) ? xrow[k0 + 2 * j] : 0u;
      const uint32_t hi = (k0 + 2 * j + 1 < K) ? xrow[k0 + 2 * j + 1] : 0u;
      out[j] = lo | (hi << 16);
    }
  }
}

// acc += W-chunk . x-chunk for one weight row and one activation row.
template <int KIND>
__device__ __forceinline__ float chunk_dot(const u32x4& wv, const uint32_t (&xv)[Layout<KIND>::kXDwords],
                                           float acc) {
  const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
  if constexpr (KIND == kBf16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = dot2_bf16(wd[j], xv[j], acc);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc = dot2_bf16(i8pair_to_bf16x2(wd[j], 0), xv[2 * j], acc);
      acc = dot2_bf16(i8pair_to_bf16x2(wd[j], 16), xv[2 * j + 1], acc);
    }
  }
  return acc;
}

template <int KIND, int MT, int ROWS, int WAVES, bool VEC>
__global__ __launch_bounds__(WAVES * kWave) void skinny_dot_kernel(const uint16_t* __restrict__ x,
                                                                   const uint8_t* __restrict__ w,
                                                                   const void* __restrict__ scale, int scale_dt,
                                                                   uint16_t* __restrict__ y,
                                                                   float* __restrict__ ws, int M, int64_t N,
                                                                   int64_t K, int split) {
  using L = Layout<KIND>;
  constexpr int P = ROWS * MT;                    // partial sums per lane
  constexpr int PL = P >= kWave ? P / kWave : 1;  // totals a lane holds after the wave reduction
  __shared__ float red[WAVES][P];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * ROWS;
  const int s = blockIdx.y;
  const int64_t nch = (K + L::kChunk - 1) / L::kChunk;
  const int64_t c_lo = s * nch / split;
  const int64_t c_hi = (s + 1) * nch / split;

  float acc[P];
#pragma unroll
  for (int p = 0; p < P; ++p) acc[p] = 0.f;

  for (int64_t c = c_lo + wave; c < c_hi; c += WAVES) {
    const int64_t k0 = c * L::kChunk + static_cast<int64_t>(lane) * L::kEpl;
    const bool kin = k0 < K;
    u32x4 wv[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      wv[r] = u32x4{0u, 0u, 0u, 0u};
      if (kin && row0 + r < N) wv[r] = load_w<KIND, VEC>(w, row0 + r, K, k0);
    }
    uint32_t xv[MT][L::kXDwords];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
      for (int j = 0; j < L::kXDwords; ++j) xv[m][j] = 0u;
      if (kin && m < M) load_x<KIND, VEC>(x + static_cast<int64_t>(m) * K, K, k0, xv[m]);
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[r * MT + m] = chunk_dot<KIND>(wv[r], xv[m], acc[r * MT + m]);
  }

  wave_transpose_reduce<P>(acc, lane);

  // Lane l now holds the wave totals of indices [l*PL, l*PL + PL) (P >= 64) or of index l / (64 / P).
  if constexpr (P >= kWave) {
#pragma unroll
    for (int j = 0; j < PL; ++j) red[wave][lane * PL + j] = acc[j];
  } else {
    if ((lane & (kWave / P - 1)) == 0) red[wave][lane / (kWave / P)] = acc[0];
  }
  __syncthreads();

  for (int p = threadIdx.x; p < P; p += WAVES * kWave) {
    const int r = p / MT;
    const int m = p % MT;
    const int64_t row = row0 + r;
    if (m >= M || row >= N) continue;
    float t = red[0][p];
#pragma unroll
    for (int v = 1; v < WAVES; ++v) t += red[v][p];
    if (split == 1) {
      if constexpr (KIND == kInt8) t *= load_scale(scale, row, scale_dt);
      y[static_cast<int64_t>(m) * N + row] = float_to_bf16_bits(t);
    } else {
      ws[(static_cast<int64_t>(s) * M + m) * N + row] = t;
    }
  }
}

// Compiled menu: a (ROWS, WAVES) pair exists for a (KIND, MT) when its register estimate fits the budget that
// WAVES leaves per wave (WAVES <= 8, at most 2 waves of the workgroup per SIMD: about 200 VGPRs; 16 waves, 4 per
// SIMD: about 100, below the 128 that a 1024-thread workgroup allows). ROWS = 2 exists for every MT at every
// WAVES <= 8, so one K order (one WAVES value) can serve every activation-row bucket of a shape.
template <int KIND, int MT, int ROWS, int WAVES>
constexpr bool menu_has() {
  constexpr int xd = Layout<KIND>::kXDwords;
  constexpr int est = ROWS * MT + ROWS * 4 + MT * xd + (KIND == kInt8 ? ROWS * 2 : 0);
  return est <= (WAVES <= 8 ? 200 : 100);
}

template <int KIND, int MT, int ROWS, int WAVES>
SkinnyFn pick_vec() {
  if constexpr (menu_has<KIND, MT, ROWS, WAVES>()) {
    return &skinny_dot_kernel<KIND, MT, ROWS, WAVES, true>;
  } else {
    return nullptr;
  }
}

template <int KIND, int MT, int ROWS>
SkinnyFn pick_waves(int waves) {
  switch (waves) {
    case 1: return pick_vec<KIND, MT, ROWS, 1>();
    case 2: return pick_vec<KIND, MT, ROWS, 2>();
    case 4: return pick_vec<KIND, MT, ROWS, 4>();
    case 8: return pick_vec<KIND, MT, ROWS, 8>();
    case 16: return pick_vec<KIND, MT, ROWS, 16>();
    default: return nullptr;
  }
}

// The element-load (unaligned / ragged K) variant exists in one shape per (KIND, MT): 4 rows x 4 waves.
constexpr int kGenericRows = 4;
constexpr int kGenericWaves = 4;

// Kernel for (KIND, MT, rows, waves); vec = false returns the element-load variant (rows/waves ignored).
template <int KIND, int MT>
SkinnyFn skinny_pick(int rows, int waves, bool vec) {
  if (!vec) return &skinny_dot_kernel<KIND, MT, kGenericRows, kGenericWaves, false>;
  switch (rows) {
    case 2: return pick_waves<KIND, MT, 2>(waves);
    case 4: return pick_waves<KIND, MT, 4>(waves);
    case 8: return pick_waves<KIND, MT, 8>(waves);
    case 16: return pick_waves<KIND, MT, 16>(waves);
    case 32: return pick_waves<KIND, MT, 32>(waves);
    default: return nullptr;
  }
}

}  // namespace bp
