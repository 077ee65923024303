// Skinny matmul with int4 group-128 weights (the tile-major format of byteprof's skinny kernels), gfx950:
// y[M, N] (bf16) = x[M, K] (bf16) . deq(W)^T for 1..16 activation rows, fp32 accumulation.
//
// Format: packed uint8 [T = ceil(N / R), G = K / 128, R, 64]: the R rows of row tile t and group g form one
// contiguous block of R x 64 bytes, and byte j of a row's group holds code j in its low nibble and code j + 64 in its
// high nibble (codes 0..15); scale [G, N] (bf16, fp16 or fp32) and zero [G, N] (fp16) per group and row;
// deq(W)[n, 128 g + j] = scale[g, n] * (code - zero[g, n]). Padding rows of the last tile are never stored.
//
// Work decomposition (every weight byte is read once):
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

namespace bp {

using Int4Fn = void (*)(const uint16_t*, const uint8_t*, const void*, int, const uint16_t*, uint16_t*, float*, int,
                        int64_t, int64_t, int);

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
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * R;
  const int64_t G = K / 128;
  const int s = blockIdx.y;
  const int64_t g_lo = s * G / split;
  const int64_t g_hi = (s + 1) * G / split;
  const uint8_t* tile = w + static_cast<int64_t>(blockIdx.x) * G * R * 64 + rr * 64 + q * 16;

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
