// Skinny matmul with int4 group-128 weights (the tile-major format of byteprof's skinny kernels), gfx950:
// y[M, N] (bf16) = x[M, K] (bf16) . deq(W)^T for 1..16 activation rows, fp32 accumulation.
//
// Format: packed uint8 [T = ceil(N / R), G = K / 128, R, 64]: the R rows of row tile t and group g form one
// contiguous block of R x 64 bytes, and byte j of a row's group holds code j in its low nibble and code j + 64 in its
// high nibble (codes 0..15); scale [G, N] (bf16, fp16 or fp32) and zero [G, N] (fp16) per group and row;
// deq(W)[n, 128 g + j] = scale[g, n] * (code - zero[g, n]). Padding rows of the last tile are never stored.
//
// Two kernels, each with one summation order per (K, WAVES, split): the matrix-core kernel (skinny_int4_mf_kernel,
// below) wherever N % 4 == 0 and scale / zero are aligned to four elements, its cost nearly flat in M; else the
// VALU kernel described next, whose work grows with every activation row.
//
// VALU kernel. Work decomposition (every weight byte is read once):
//   - a workgroup owns one row tile (R = 16, 32 or 64 rows) and WAVES waves; the tile's groups are dealt to the waves
//     (with split > 1, consecutive group ranges go to separate workgroups and a fixed-order reduce adds them);
//   - a group of 16 rows is one fully coalesced 1 KiB load: lane (rr = lane / 4, q = lane % 4) reads 16 bytes of row
//     rr, i.e. low-nibble codes 16 q .. 16 q + 15 and high-nibble codes 64 + 16 q .. 64 + 16 q + 15;
//   - codes become bf16 operands without arithmetic: v_perm_b32 puts a code q (a byte below 128) under the byte 0x43,
//     which is bf16(128 + q) exactly (bit 7 of the low byte is the exponent's lowest bit, so the byte must stay below
//     128: the high nibbles are shifted down first); the products go through v_dot2_f32_bf16 into fp32 and the offset
//     is removed per group with the lane's own sums of the same activations:
//     sum (q - z) x = (d_lo - 128 X_lo) + (d_hi - 128 X_hi) - z (X_lo + X_hi);
//   - each lane applies its rows' scale and zero to its own partial sums, so no reduction happens inside the loop; at
//     the end the four lanes of a row are added (DPP), then the waves in LDS in wave order.
// Unlike the reference's tensor-core path (skinny.py:46-63), which rounds q - zero to bf16 before the product, the
// codes, the zero and the activations enter the sums exactly (closer to the dequantize-then-matmul result). The
// order of every sum depends on (K, WAVES, split) only, so an output row does not depend on M (bitwise).
//
// Reference semantics: byteprof/optim/skinny.py:46-63 (MODE 3 kernel), :172-217 (quantize_int4, pack_int4,
// unpack_int4, dequantize), used through skinny_mm (skinny.py:136-166) and SkinnyLinear int4_wo
// (skinny_linear.py:39-44).

#include "byteprof_amd.h"
#include "common.h"
#include "skinny_mf_kernel.h"  // MfPro and mf_prologue: the norm prologue the matrix-core kernels share

namespace bp {

using Int4Fn = void (*)(const uint16_t*, const uint8_t*, const void*, int, const uint16_t*, uint16_t*, float*, int,
                        int64_t, int64_t, int);
using Int4MfFn = void (*)(const uint16_t*, const uint8_t*, const void*, int, const uint16_t*, uint16_t*, float*, int,
                          int64_t, int64_t, int, MfPro);

namespace {

constexpr uint32_t kBf16Exp128 = 0x43434343u;  // 0x43 in every byte: bf16 0x43xx = 128 + xx
constexpr uint32_t kBf16OnePair = 0x3F803F80u; // two bf16 1.0

// Four codes (bytes of m, each below 128) as two bf16 pairs (128 + byte).
__device__ __forceinline__ void codes_to_bf16(uint32_t m, uint32_t& p01, uint32_t& p23) {
  // v_perm_b32 (S0 = m: bytes 4..7, S1 = 0x43434343: bytes 0..3): result bytes [m0, 0x43, m1, 0x43] / [m2, .., m3, ..]
  p01 = __builtin_amdgcn_perm(m, kBf16Exp128, 0x00050004u);
  p23 = __builtin_amdgcn_perm(m, kBf16Exp128, 0x00070006u);
}

template <int MT, int RB, int WAVES>
__global__ __launch_bounds__(WAVES * kWave) void skinny_int4_kernel(const uint16_t* __restrict__ x,
                                                                    const uint8_t* __restrict__ w,
                                                                    const void* __restrict__ scale, int scale_dt,
                                                                    const uint16_t* __restrict__ zero,
                                                                    uint16_t* __restrict__ y,
                                                                    float* __restrict__ ws, int M, int64_t N,
                                                                    int64_t K, int split) {
  constexpr int R = 16 * RB;
  __shared__ float red[WAVES][R][MT];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int rr = lane >> 2;
  const int q = lane & 3;
  const int64_t tb = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t n0 = tb * R;
  const int64_t G = K / 128;
  const int s = blockIdx.y;
  const int64_t g_lo = s * G / split;
  const int64_t g_hi = (s + 1) * G / split;
  const uint8_t* tile = w + tb * G * R * 64 + rr * 64 + q * 16;

  // this lane's rows n0 + 16 h + rr (rows past N: clamped for the scale / zero reads, never stored)
  int64_t nrow[RB];
#pragma unroll
  for (int h = 0; h < RB; ++h) nrow[h] = min(n0 + 16 * h + rr, N - 1);

  float acc[RB][MT];
#pragma unroll
  for (int h = 0; h < RB; ++h)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[h][m] = 0.f;

  for (int64_t g = g_lo + wave; g < g_hi; g += WAVES) {
    u32x4 wv[RB];
#pragma unroll
    for (int h = 0; h < RB; ++h)
      wv[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + (g * R + 16 * h) * 64));
    float sc[RB], zf[RB];
#pragma unroll
    for (int h = 0; h < RB; ++h) {
      sc[h] = load_scale(scale, g * N + nrow[h], scale_dt);
      zf[h] = static_cast<float>(__builtin_bit_cast(_Float16, zero[g * N + nrow[h]]));
    }
    // bf16 operand pairs (128 + code) of the codes: lo[h][p] = codes 16 q + 2p, +1; hi[h][p] = codes 64 + 16 q + 2p, +1
    uint32_t lo[RB][8], hi[RB][8];
#pragma unroll
    for (int h = 0; h < RB; ++h) {
      const uint32_t d[4] = {wv[h].x, wv[h].y, wv[h].z, wv[h].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        codes_to_bf16(d[k] & 0x0F0F0F0Fu, lo[h][2 * k], lo[h][2 * k + 1]);
        codes_to_bf16((d[k] >> 4) & 0x0F0F0F0Fu, hi[h][2 * k], hi[h][2 * k + 1]);
      }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m >= M) continue;
      const uint16_t* xr = x + static_cast<int64_t>(m) * K + g * 128 + q * 16;
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(xr), a1 = *reinterpret_cast<const u32x4*>(xr + 8);
      const u32x4 b0 = *reinterpret_cast<const u32x4*>(xr + 64), b1 = *reinterpret_cast<const u32x4*>(xr + 72);
      const uint32_t xl[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      const uint32_t xh[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
      float sl = 0.f, sh = 0.f;
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        sl = dot2_bf16(xl[p], kBf16OnePair, sl);
        sh = dot2_bf16(xh[p], kBf16OnePair, sh);
      }
#pragma unroll
      for (int h = 0; h < RB; ++h) {
        float dl = 0.f, dh = 0.f;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          dl = dot2_bf16(lo[h][p], xl[p], dl);
          dh = dot2_bf16(hi[h][p], xh[p], dh);
        }
        const float part = (dl - 128.f * sl) + (dh - 128.f * sh) - zf[h] * (sl + sh);
        acc[h][m] += sc[h] * part;
      }
    }
  }

  // the row's four lanes, then the waves in wave order
#pragma unroll
  for (int h = 0; h < RB; ++h)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float v = acc[h][m];
      v += dpp_f32<0xB1, 0xF>(v);  // quad_perm [1,0,3,2]
      v += dpp_f32<0x4E, 0xF>(v);  // quad_perm [2,3,0,1]
      if (q == 0) red[wave][16 * h + rr][m] = v;
    }
  __syncthreads();
  for (int e = threadIdx.x; e < R * MT; e += WAVES * kWave) {
    const int row = e / MT;
    const int m = e % MT;
    const int64_t n = n0 + row;
    if (m >= M || n >= N) continue;
    float t = red[0][row][m];
#pragma unroll
    for (int v = 1; v < WAVES; ++v) t += red[v][row][m];
    if (split == 1)
      y[static_cast<int64_t>(m) * N + n] = float_to_bf16_bits(t);
    else
      ws[(static_cast<int64_t>(s) * M + m) * N + n] = t;
  }
}

// ---- matrix-core form -----------------------------------------------------------------------------------------
// v_mfma_f32_16x16x32_bf16 with a block of 16 weight rows as A and the activation rows (up to 16, zero-padded) as
// the B columns, so the work per group does not grow with M. Lane l (row / column i = l % 16, K block kb = l / 16)
// loads bytes 16 kb .. 16 kb + 15 of row i of a block's 1 KiB (one load covers the block), i.e. codes 16 kb + e (low
// nibbles) and 64 + 16 kb + e (high nibbles), e < 16, and the activations at the same K indices; the four MFMAs of a
// group take K slots {16 kb + e}, {16 kb + 8 + e}, {64 + 16 kb + e}, {64 + 16 kb + 8 + e} (e < 8) of every kb, the
// same for A and B, so D[r][m] is the group's sum over all 128 codes. (Loading the block in lane order and passing
// it across lanes with ds_bpermute, consecutive lanes on consecutive bytes, was 1.4 us slower on the LM head.)
// Codes enter as bf16(128 + code) (v_perm_b32 under 0x43); per group, D (a fresh accumulator) becomes
// scale (D - (128 + zero) X), X the group's sum of the activation row (four more MFMAs: an all-ones A against the
// same B operands), and the lane adds it to its rows' sums in group order; the waves'
// sums meet in LDS in wave order. The groups of a wave are loaded DEPTH ahead of their use. A group's scales and
// zeros for the tile's rows (its record: two 32..128-byte pieces of the [G, N] layout) arrive with the group's
// loads as one dword per lane (two at 64 rows in fp32) and pass through the wave's own LDS stage to the lanes that
// use them: loaded per lane, 4 rows at a time, they were twice as many small scattered loads and cost as much as the
// weights' own stream (the LM head at one row: 32.9 us with them, 23.6 us without). The order of every sum depends
// on (K, WAVES, split) only: an output row does not depend on M (bitwise).
// Needs N % 4 == 0 (every dword of a record is whole, and a lane's four D rows read their scales and zeros as one
// 8- or 16-byte LDS read) and 16-byte aligned x, 8-byte aligned zero, scale aligned to 4 of its elements.

template <int RB, int NR>
struct I4Slot {
  u32x4 wv[RB];      // bytes 16 l .. 16 l + 15 of each 16-row block (lane order)
  u32x4 xv[4];       // activations at K 16 kb + 0..7, + 8..15, 64 + 16 kb + 0..7, + 8..15 of the lane's column
  uint32_t rv[NR];   // dwords 64 c + l of the group's record
};

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

using u32x2 = unsigned __attribute__((ext_vector_type(2)));

// PRO (up to 8 activation rows, split 1): the rows staged in LDS with gamma, the residual rows and gamma2 (dynamic
// shared memory, (2 M + 2) K bf16), transformed by mf_prologue (the norm kernel's arithmetic: the product equals a norm launch
// followed by the plain kernel, bit for bit) while the first groups' weights are in flight; the B operands are then
// read from LDS.
template <int RB, int WAVES, int DEPTH, int SDT, int EPI = 0, bool PRO = false>
__global__ __launch_bounds__(WAVES * kWave) void skinny_int4_mf_kernel(const uint16_t* __restrict__ x,
                                                                       const uint8_t* __restrict__ w,
                                                                       const void* __restrict__ scale, int scale_dt,
                                                                       const uint16_t* __restrict__ zero,
                                                                       uint16_t* __restrict__ y,
                                                                       float* __restrict__ ws, int M, int64_t N,
                                                                       int64_t K, int split, MfPro pro) {
  using floatx4 = float __attribute__((ext_vector_type(4)));
  using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
  constexpr int R = 16 * RB;
  __shared__ float red[WAVES][R][16];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // uniform: the group loop is scalar
  const int i = lane & 15, kb = lane >> 4;
  const int64_t tb = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t n0 = tb * R;
  const int64_t G = K / 128;
  const int s = blockIdx.y;
  const int64_t g_lo = s * G / split;
  const int64_t g_hi = (s + 1) * G / split;
  const int64_t first = g_lo + wave;
  const int cnt = first < g_hi ? static_cast<int>((g_hi - first + WAVES - 1) / WAVES) : 0;
  const uint8_t* tile = w + tb * G * R * 64 + i * 64 + kb * 16;
  // the activations through one buffer resource (the launch takes this kernel for K < 2^24: 2 M K < 2^31 bytes);
  // a column past M has an offset past it, so its loads return zeros without a memory request
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(x, static_cast<int>(2 * M * K));
  const uint32_t xoff = i < M ? static_cast<uint32_t>(2 * (i * K + kb * 16)) : 0x80000000u;
  constexpr bool f32 = SDT == BP_DT_F32;  // the scale's dtype (scale_dt == SDT)

  // a group's record: [R scales (scale dtype) | R zeros (fp16)] of the tile's rows, kRecDw dwords; lane l holds
  // dwords 64 c + l (lanes past the record repeat its last dword); rows past N read row N - 2 of the group (never
  // stored). Dword 64 c + l sits at rsrc[c] + g * rstride[c] for group g.
  constexpr int SEB = f32 ? 4 : 2;
  constexpr int kScDw = R * SEB / 4, kRecDw = kScDw + R / 2;  // dwords of a record's scales / of the whole record
  constexpr int kRecLoads = (kRecDw + kWave - 1) / kWave;
  __shared__ __attribute__((aligned(16))) uint32_t stage[WAVES][kRecLoads * kWave];
  const uint8_t* rsrc[kRecLoads];
  int64_t rstride[kRecLoads];
#pragma unroll
  for (int c = 0; c < kRecLoads; ++c) {
    const int p = min(c * kWave + lane, kRecDw - 1);
    if (p < kScDw) {
      const int64_t r0 = n0 + p * 4 / SEB;
      rsrc[c] = static_cast<const uint8_t*>(scale) + (r0 < N ? r0 : N - 4 / SEB) * SEB;
      rstride[c] = N * SEB;
    } else {
      const int64_t r0 = n0 + 2 * (p - kScDw);
      rsrc[c] = reinterpret_cast<const uint8_t*>(zero + (r0 < N ? r0 : N - 2));
      rstride[c] = N * 2;
    }
  }

  extern __shared__ __attribute__((aligned(16))) uint16_t i4_xs[];  // PRO: [x row | gamma | residual | gamma2]
  __shared__ float pro_sums[PRO ? 8 : 1];
  auto load = [&](I4Slot<RB, kRecLoads>& sl, int j) {
    const int64_t g = first + static_cast<int64_t>(j) * WAVES;
#pragma unroll
    for (int h = 0; h < RB; ++h)
      sl.wv[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + (g * R + 16 * h) * 64));
    if constexpr (!PRO) {
      const uint32_t xo = xoff + static_cast<uint32_t>(256 * g);
      sl.xv[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, xo, 0, 0));
      sl.xv[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, xo + 16, 0, 0));
      sl.xv[2] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, xo + 128, 0, 0));
      sl.xv[3] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, xo + 144, 0, 0));
    }
#pragma unroll
    for (int c = 0; c < kRecLoads; ++c) sl.rv[c] = *reinterpret_cast<const uint32_t*>(rsrc[c] + g * rstride[c]);
  };

  float acc[RB][4];
#pragma unroll
  for (int h = 0; h < RB; ++h)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[h][r] = 0.f;

  uint32_t* st = stage[wave];
  auto compute = [&](const I4Slot<RB, kRecLoads>& sl, int j) {
    const u32x4* xv = sl.xv;
    u32x4 xl[4];
    if constexpr (PRO) {
      // the transformed rows from LDS (columns past M zeros, never stored)
      const bool live = i < M;
      const uint16_t* src =
          i4_xs + (live ? i : 0) * K + (first + static_cast<int64_t>(j) * WAVES) * 128 + kb * 16;
      const u32x4 zv = u32x4{0u, 0u, 0u, 0u};
      xl[0] = live ? *reinterpret_cast<const u32x4*>(src) : zv;
      xl[1] = live ? *reinterpret_cast<const u32x4*>(src + 8) : zv;
      xl[2] = live ? *reinterpret_cast<const u32x4*>(src + 64) : zv;
      xl[3] = live ? *reinterpret_cast<const u32x4*>(src + 72) : zv;
      xv = xl;
    }
    // the record through the wave's stage (the wave's LDS operations run in order: the previous group's reads are
    // done before these writes land)
#pragma unroll
    for (int c = 0; c < kRecLoads; ++c) st[c * kWave + lane] = sl.rv[c];
    __builtin_amdgcn_wave_barrier();
    // columns past M hold zeros: computed, never stored
    const u32x4 ones = u32x4{kBf16OnePair, kBf16OnePair, kBf16OnePair, kBf16OnePair};
    // X: the group's sum of each column's activations, as the product of an all-ones A with the same B operands
    floatx4 X = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      X = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ones), __builtin_bit_cast(bf16x8, xv[c]),
                                                  X, 0, 0, 0);
#pragma unroll
    for (int h = 0; h < RB; ++h) {
      const uint32_t d[4] = {sl.wv[h].x, sl.wv[h].y, sl.wv[h].z, sl.wv[h].w};
      // operand c: codes of dwords 2 (c % 2), 2 (c % 2) + 1, low nibbles for c < 2, high for c >= 2
      u32x4 a[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int sh = c < 2 ? 0 : 4;
        uint32_t p0, p1, p2, p3;
        codes_to_bf16((d[2 * (c % 2)] >> sh) & 0x0F0F0F0Fu, p0, p1);
        codes_to_bf16((d[2 * (c % 2) + 1] >> sh) & 0x0F0F0F0Fu, p2, p3);
        a[c] = u32x4{p0, p1, p2, p3};
      }
      floatx4 D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c)
        D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[c]),
                                                    __builtin_bit_cast(bf16x8, xv[c]), D, 0, 0, 0);
      // the lane's four D rows 16 h + 4 kb + r of the group: their scales and zeros from the record
      const int rr = 16 * h + 4 * kb;
      const u32x2 zq = *reinterpret_cast<const u32x2*>(st + kScDw + rr / 2);
      uint32_t sw[4];
      if constexpr (f32) {
        const u32x4 sq = *reinterpret_cast<const u32x4*>(st + rr);
        sw[0] = sq.x, sw[1] = sq.y, sw[2] = sq.z, sw[3] = sq.w;
      } else {
        const u32x2 sq = *reinterpret_cast<const u32x2*>(st + rr / 2);
        sw[0] = sq.x, sw[1] = sq.y, sw[2] = 0u, sw[3] = 0u;
      }
      const uint32_t zw[2] = {zq.x, zq.y};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float z = half_bits_to_float(r % 2 == 0 ? zw[r / 2] & 0xffffu : zw[r / 2] >> 16);
        const uint32_t s16 = r % 2 == 0 ? sw[r / 2] & 0xffffu : sw[r / 2] >> 16;
        const float sc = f32 ? __uint_as_float(sw[r]) : (SDT == BP_DT_BF16 ? bf16_bits_to_float(s16)
                                                                             : half_bits_to_float(s16));
        acc[h][r] += sc * (D[r] - (128.f + z) * X[r]);
      }
    }
  };

  // rounds of DEPTH groups with every load unconditional, so the waits count exactly (a load past the wave's last
  // group reloads it, unused), and no peeled rest: the slots are not live after the loop, so the first round's
  // loads land in the registers the loop uses
  I4Slot<RB, kRecLoads> sl[DEPTH];
  if constexpr (PRO) {
    // the rows, gamma, the residual rows and gamma2 straight into LDS (64 lanes x 16 bytes per load), ahead of the
    // first groups' weights; every wave takes part in the prologue's barriers, groups or not
    const int kn = static_cast<int>(K);
    uint16_t* gl = i4_xs + M * kn;
    uint16_t* dst2 = gl + (pro.residual != nullptr ? 1 + M : 1) * kn;
    for (int c = wave; c * 512 < kn; c += WAVES) {
      const int e = c * 512 + 8 * lane;
      if (e < kn) {
        for (int m = 0; m < M; ++m)
          __builtin_amdgcn_global_load_lds(as_global(x + static_cast<int64_t>(m) * kn + e),
                                           (__attribute__((address_space(3))) void*)(i4_xs + m * kn + c * 512), 16,
                                           0, 0);
        if (pro.kind == BP_PRO_NORM) {
          __builtin_amdgcn_global_load_lds(as_global(pro.gamma + e),
                                           (__attribute__((address_space(3))) void*)(gl + c * 512), 16, 0, 0);
          if (pro.residual != nullptr)
            for (int m = 0; m < M; ++m)
              __builtin_amdgcn_global_load_lds(
                  as_global(pro.residual + static_cast<int64_t>(m) * kn + e),
                  (__attribute__((address_space(3))) void*)(gl + (1 + m) * kn + c * 512), 16, 0, 0);
          if (pro.gamma2 != nullptr)
            __builtin_amdgcn_global_load_lds(as_global(pro.gamma2 + e),
                                             (__attribute__((address_space(3))) void*)(dst2 + c * 512), 16, 0, 0);
        }
      }
    }
    if (cnt > 0) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        load(sl[d], d < cnt ? d : cnt - 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // the staged operands (and the first groups) have landed
    __syncthreads();
    mf_prologue<WAVES * kWave>(i4_xs, M, kn, pro, blockIdx.x == 0 && blockIdx.y == 0,
                               pro.kind == BP_PRO_NORM ? gl : nullptr, pro_sums);
  } else if (cnt > 0) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      load(sl[d], d < cnt ? d : cnt - 1);
      __builtin_amdgcn_sched_barrier(0);  // the slots' loads in slot order
    }
  }
  if (cnt > 0) {
    for (int j0 = 0; j0 < cnt; j0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int j = j0 + d;
        if (j < cnt) compute(sl[d], j);
        load(sl[d], j + DEPTH < cnt ? j + DEPTH : cnt - 1);
        __builtin_amdgcn_sched_barrier(0);  // keeps the pipeline's order: group j's arithmetic before j + 1's
      }
    }
  }

  // the waves' sums in wave order
#pragma unroll
  for (int h = 0; h < RB; ++h)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][16 * h + 4 * kb + r][i] = acc[h][r];
  __syncthreads();
  const auto total = [&](int row, int m) {
    float t = red[0][row][m];
#pragma unroll
    for (int v = 1; v < WAVES; ++v) t += red[v][row][m];
    return t;
  };
  if constexpr (EPI == 0) {
    for (int e = threadIdx.x; e < R * 16; e += WAVES * kWave) {
      const int row = e / 16;
      const int m = e % 16;
      const int64_t n = n0 + row;
      if (m >= M || n >= N) continue;
      const float t = total(row, m);
      if (split == 1)
        y[static_cast<int64_t>(m) * N + n] = float_to_bf16_bits(t);
      else
        ws[(static_cast<int64_t>(s) * M + m) * N + n] = t;
    }
  } else {
    // the gate|up SiLU product (split 1): rows 2f and 2f + 1 of the tile are the gate and up rows of output f,
    // y [M, N / 2]; the arithmetic of bp_decode_silu_mul_rows on the rounded sums
    for (int e = threadIdx.x; e < (R / 2) * 16; e += WAVES * kWave) {
      const int row = 2 * (e / 16);
      const int m = e % 16;
      const int64_t n = n0 + row;
      if (m >= M || n + 1 >= N) continue;
      const float gb = round_to_bf16(total(row, m));
      const float a = round_to_bf16(gb / (1.f + expf(-gb)));
      y[static_cast<int64_t>(m) * (N / 2) + n / 2] = float_to_bf16_bits(a * round_to_bf16(total(row + 1, m)));
    }
  }
}

template <int RB, int DEPTH, int SDT, int EPI, bool PRO>
Int4MfFn int4_mf_waves(int waves) {
  switch (waves) {
    case 1: return &skinny_int4_mf_kernel<RB, 1, DEPTH, SDT, EPI, PRO>;
    case 2: return &skinny_int4_mf_kernel<RB, 2, DEPTH, SDT, EPI, PRO>;
    case 4: return &skinny_int4_mf_kernel<RB, 4, DEPTH, SDT, EPI, PRO>;
    case 8: return &skinny_int4_mf_kernel<RB, 8, DEPTH, SDT, EPI, PRO>;
    default: return nullptr;
  }
}

// the prologue variants for bf16 scales only (quantize_int4 keeps the weights' dtype, bf16 in a decoder)
template <int RB, int DEPTH, int EPI, bool PRO>
Int4MfFn int4_mf_dtype(int waves, int scale_dt) {
  switch (scale_dt) {
    case BP_DT_BF16: return int4_mf_waves<RB, DEPTH, BP_DT_BF16, EPI, PRO>(waves);
    case BP_DT_F16:
      if constexpr (!PRO) return int4_mf_waves<RB, DEPTH, BP_DT_F16, EPI, false>(waves);
      return nullptr;
    case BP_DT_F32:
      if constexpr (!PRO) return int4_mf_waves<RB, DEPTH, BP_DT_F32, EPI, false>(waves);
      return nullptr;
    default: return nullptr;
  }
}

template <int EPI, bool PRO>
Int4MfFn int4_mf_tile(int tile_rows, int waves, int scale_dt) {
  switch (tile_rows) {
    case 16: return int4_mf_dtype<1, 4, EPI, PRO>(waves, scale_dt);
    case 32: return int4_mf_dtype<2, 3, EPI, PRO>(waves, scale_dt);
    case 64: return int4_mf_dtype<4, 2, EPI, PRO>(waves, scale_dt);
    default: return nullptr;
  }
}

template <int MT, int RB>
Int4Fn int4_waves(int waves) {
  switch (waves) {
    case 1: return &skinny_int4_kernel<MT, RB, 1>;
    case 2: return &skinny_int4_kernel<MT, RB, 2>;
    case 4: return &skinny_int4_kernel<MT, RB, 4>;
    case 8: return &skinny_int4_kernel<MT, RB, 8>;
    default: return nullptr;
  }
}

template <int MT>
Int4Fn int4_rows(int rb, int waves) {
  switch (rb) {
    case 1: return int4_waves<MT, 1>(waves);
    case 2: return int4_waves<MT, 2>(waves);
    case 4: return int4_waves<MT, 4>(waves);
    default: return nullptr;
  }
}

}  // namespace

// Matrix-core kernel for (tile rows, waves, scale dtype, epilogue: 0 the product, 1 the gate|up SiLU product,
// prologue), or null; groups in flight per wave: 4 at 16 tile rows, 3 at 32, 2 at 64.
Int4MfFn int4_mf_pick(int tile_rows, int waves, int scale_dt, int epi, bool pro) {
  if (pro)
    return epi == 0 ? int4_mf_tile<0, true>(tile_rows, waves, scale_dt)
                    : int4_mf_tile<1, true>(tile_rows, waves, scale_dt);
  return epi == 0 ? int4_mf_tile<0, false>(tile_rows, waves, scale_dt)
                  : int4_mf_tile<1, false>(tile_rows, waves, scale_dt);
}

// Kernel for (activation-row bucket, tile rows, waves), or null.
Int4Fn int4_pick(int mt, int tile_rows, int waves) {
  if (tile_rows <= 0 || tile_rows % 16 != 0) return nullptr;
  const int rb = tile_rows / 16;
  switch (mt) {
    case 1: return int4_rows<1>(rb, waves);
    case 2: return int4_rows<2>(rb, waves);
    case 4: return int4_rows<4>(rb, waves);
    case 8: return int4_rows<8>(rb, waves);
    case 16: return int4_rows<16>(rb, waves);
    default: return nullptr;
  }
}

}  // namespace bp
