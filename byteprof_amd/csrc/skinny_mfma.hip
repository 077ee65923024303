// Skinny weight-only matmul on the matrix cores (v_mfma_f32_16x16x32_bf16), gfx950: y[M, N] = x[M, K] . W[N, K]^T
// for 1..16 activation rows, bf16 activations, fp32 accumulation, bf16 output; weights bf16, or int8 with one scale
// per output row (converted exactly to bf16 in registers, the scale applied to the fp32 sum).
//
// The operands are swapped against the usual GEMM tiling: the MFMA's A operand is a block of 16 weight rows (output
// channels) and its B operand the activation rows (B column j = activation row j, zero for j >= M), so one
// 16 x 16 x 32 MFMA advances 16 output channels x 16 activation rows by 32 K. At the verify widths (M = 8..16) this
// does in one instruction what the VALU kernel does in M x 16 v_dot2 per lane; at M = 1 the same instruction count
// streams the same weight bytes, 15 of its 16 columns idle.
//
// Work decomposition (HBM-bound; every weight byte is read exactly once):
//   - a workgroup owns RB blocks of 16 consecutive weight rows and WAVES wavefronts; K is cut into steps of 128
//     (bf16) or 256 (int8) elements; step t of the workgroup's K range goes to wave t % WAVES;
//   - in a step, lane (i = lane % 16, g = lane / 16) of a wave loads 64 bytes of weight row i of each block with
//     four 16-byte non-temporal loads, load q reading bytes [64 q + 16 g, 64 q + 16 g + 16) of the step's 256 bytes
//     of that row: the four lanes of a row read 64 contiguous bytes per load instruction. The lane's activation
//     operand holds x[i][k] for the same k's, so A's and B's K indices agree lane by lane (a contraction does not
//     care which K each lane slot carries, as long as both operands carry the same one);
//   - each block accumulates a 16 x 16 fp32 tile in 4 registers per lane (lane l: activation row l % 16, output
//     channels 4 (l / 16) .. + 3); the wave tiles are added in LDS in wave order, then scaled, rounded and stored;
//   - with split > 1, grid.y workgroups take consecutive step ranges and store fp32 partials (added in split order
//     by splitk_reduce in skinny.hip).
// The order of every sum depends on (K, WAVES, split) only, never on M or RB: output row m is bitwise independent
// of how many activation rows share the launch.
//
// Reference semantics: byteprof/optim/skinny.py:36-90 (the kernel's bf16 / int8 modes and split reduce), used by
// skinny_mm (skinny.py:136-166) at the speculative-verify widths (activation rows 5..16 of the sweep M in
// {1, 2, 4, 8, 16}).

#include "byteprof_amd.h"
#include "skinny_kernel.h"

namespace bp {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int KIND>
struct MfmaLayout {
  static constexpr int kElemBytes = KIND == kBf16 ? 2 : 1;
  static constexpr int kLoadElems = 16 / kElemBytes;       // weight elements per lane per 16-byte load
  static constexpr int kStep = 4 * 4 * kLoadElems;         // K per step: 4 loads x 4 lanes per row
  static constexpr int kMfmas = 4 * kLoadElems / 8;        // MFMAs per block per step (8 K per lane each)
};

__device__ __forceinline__ floatx4 mfma_bf16(u32x4 a, u32x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// Eight int8 weights (two dwords) as eight bf16 values (exact).
__device__ __forceinline__ u32x4 i8x8_to_bf16x8(uint32_t d0, uint32_t d1) {
  return u32x4{i8pair_to_bf16x2(d0, 0), i8pair_to_bf16x2(d0, 16), i8pair_to_bf16x2(d1, 0), i8pair_to_bf16x2(d1, 16)};
}

// One step's operands of a lane: 64 weight bytes of each of its RB rows and the activations for the same K.
template <int KIND, int RB>
struct Operands {
  using L = MfmaLayout<KIND>;
  u32x4 wv[RB][4];
  u32x4 xv[L::kMfmas];

  // live = false: a placeholder step past the end, whose loads read the lane's activations instead (in bounds,
  // cached) and whose values are never used.
  __device__ __forceinline__ void load(const uint8_t* const (&wp)[RB], const uint16_t* xp, int64_t k0, bool live) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint8_t* p = live ? wp[rb] + (k0 + 4 * q * L::kLoadElems) * L::kElemBytes
                                : reinterpret_cast<const uint8_t*>(xp);
        wv[rb][q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
      }
    // activation operand j holds x[i][k] for the K indices of weight load q (k = k0 + (4 q + g) kLoadElems + e):
    // for bf16 the 8 elements of load q = j; for int8 half j % 2 of load q = j / 2
#pragma unroll
    for (int j = 0; j < L::kMfmas; ++j) {
      const int64_t kx = KIND == kBf16 ? 4 * j * L::kLoadElems : 4 * (j >> 1) * L::kLoadElems + (j & 1) * 8;
      const uint16_t* p = live ? xp + k0 + kx : xp;
      xv[j] = *reinterpret_cast<const u32x4*>(p);
    }
  }

  __device__ __forceinline__ void mma(floatx4 (&acc)[RB]) const {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if constexpr (KIND == kBf16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[rb] = mfma_bf16(wv[rb][j], xv[j], acc[rb]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[rb] = mfma_bf16(i8x8_to_bf16x8(wv[rb][q].x, wv[rb][q].y), xv[2 * q], acc[rb]);
          acc[rb] = mfma_bf16(i8x8_to_bf16x8(wv[rb][q].z, wv[rb][q].w), xv[2 * q + 1], acc[rb]);
        }
      }
    }
  }
};

// SILU: the gate|up projection with the SiLU product as the epilogue (split 1): w rows 2f / 2f + 1 are the gate /
// up rows of output f, and y [M, N / 2] receives bf16(bf16(silu(g)) * u) of the rows' bf16-rounded sums g, u (the
// rounding and formula of the decode loop's silu_mul). A lane's four channels of a tile are two such pairs.
template <int KIND, int RB, int WAVES, int DEPTH, bool SILU = false>
__global__ __launch_bounds__(WAVES * kWave) void skinny_mfma_kernel(const uint16_t* __restrict__ x,
                                                                    const uint8_t* __restrict__ w,
                                                                    const void* __restrict__ scale, int scale_dt,
                                                                    uint16_t* __restrict__ y,
                                                                    float* __restrict__ ws, int M, int64_t N,
                                                                    int64_t K, int split) {
  using L = MfmaLayout<KIND>;
  __shared__ floatx4 red[WAVES > 1 ? WAVES : 1][RB][kWave];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int i = lane & 15;
  const int g = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16 * RB;
  const int s = blockIdx.y;
  const int64_t nst = K / L::kStep;
  const int64_t t_lo = s * nst / split;
  const int64_t t_hi = (s + 1) * nst / split;

  // this lane's weight rows (rows past N read row N - 1) and activation row (rows past M read row 0): B columns
  // j >= M and A rows past N only produce tile elements that are never stored (every element of an MFMA tile
  // depends only on its own A row and B column)
  const uint8_t* wp[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int64_t row = min(n0 + 16 * rb + i, N - 1);
    wp[rb] = w + (row * K + g * L::kLoadElems) * L::kElemBytes;
  }
  const uint16_t* xp = x + static_cast<int64_t>(i < M ? i : 0) * K + g * L::kLoadElems;

  floatx4 acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = floatx4{0.f, 0.f, 0.f, 0.f};

  // DEPTH 2: two steps in flight per wave: the loads of step t + WAVES are issued before the MFMAs of step t
  // (sched_barrier keeps the scheduler from sinking them below the MFMAs). Every iteration issues the same loads
  // unconditionally (past the wave's last step they re-read this lane's activation vector, which is in cache), so
  // the compiler's wait counts stay exact.
  if constexpr (DEPTH == 2) {
    Operands<KIND, RB> buf[2];
    int64_t t = t_lo + wave;
    const int64_t mine = t < t_hi ? (t_hi - t + WAVES - 1) / WAVES : 0;  // steps of this wave
    buf[0].load(wp, xp, t * L::kStep, t < t_hi);
    for (int64_t p = 0; p + 1 < mine; p += 2) {  // steps t (buf[0]) and t + WAVES (buf[1])
      buf[1].load(wp, xp, (t + WAVES) * L::kStep, true);
      __builtin_amdgcn_sched_barrier(0);
      buf[0].mma(acc);
      t += 2 * WAVES;
      buf[0].load(wp, xp, t * L::kStep, t < t_hi);
      __builtin_amdgcn_sched_barrier(0);
      buf[1].mma(acc);
    }
    if (mine & 1) buf[0].mma(acc);
  } else {
    // one step in flight per wave; the CU's other waves cover the latency (fewer registers, more waves)
    for (int64_t t = t_lo + wave; t < t_hi; t += WAVES) {
      Operands<KIND, RB> op;
      op.load(wp, xp, t * L::kStep, true);
      op.mma(acc);
    }
  }

  if constexpr (WAVES > 1) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) red[wave][rb][lane] = acc[rb];
    __syncthreads();
  }
  // thread (rb, l): sums tile element set of lane l of block rb over the waves, in wave order
  for (int e = threadIdx.x; e < RB * kWave; e += WAVES * kWave) {
    const int rb = e / kWave;
    const int l = e % kWave;
    floatx4 t;
    if constexpr (WAVES > 1) {
      t = red[0][rb][l];
#pragma unroll
      for (int v = 1; v < WAVES; ++v) t += red[v][rb][l];
    } else {
      t = acc[0];
#pragma unroll
      for (int r = 1; r < RB; ++r)
        if (r == rb) t = acc[r];
    }
    const int m = l & 15;
    if (m >= M) continue;
    const float tv[4] = {t.x, t.y, t.z, t.w};
    if constexpr (SILU) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int64_t n = n0 + 16 * rb + 4 * (l >> 4) + 2 * p;  // even: the gate row; n + 1 the up row
        if (n + 1 >= N) continue;
        float gv = tv[2 * p], uv = tv[2 * p + 1];
        if constexpr (KIND == kInt8) {
          gv *= load_scale(scale, n, scale_dt);
          uv *= load_scale(scale, n + 1, scale_dt);
        }
        const float gb = round_to_bf16(gv);
        const float a = round_to_bf16(gb / (1.f + expf(-gb)));
        y[static_cast<int64_t>(m) * (N / 2) + n / 2] = float_to_bf16_bits(a * round_to_bf16(uv));
      }
      continue;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t n = n0 + 16 * rb + 4 * (l >> 4) + r;
      if (n >= N) continue;
      float v = tv[r];
      if (split == 1) {
        if constexpr (KIND == kInt8) v *= load_scale(scale, n, scale_dt);
        y[static_cast<int64_t>(m) * N + n] = float_to_bf16_bits(v);
      } else {
        ws[(static_cast<int64_t>(s) * M + m) * N + n] = v;
      }
    }
  }
}

// LDS-staged variant: the weights of a 16-row block are streamed in 1 KiB steps per row with fully contiguous loads
// (load r of a step reads 1 KiB of row r: the pattern of the VALU kernels, ~20% faster from HBM than 16 rows x 64
// bytes per instruction), written into a wave-private LDS buffer (rows padded to 1040 bytes so that the MFMA-layout
// reads spread over the banks) and read back as A operands. The workgroup stages its K slice of the activations (at
// most 2048 elements: split >= K / 2048) in LDS once, in bf16, rows past M never read from memory.
//
// Work: a workgroup takes rounds of c = WAVES / P blocks. Without SHARE, P = 1: each wave owns whole blocks and
// stores them itself. With SHARE, P = min(WAVES, steps per block) waves per block: wave p of a block takes the steps
// p, p + P, ... of the slice, and at the end of a round the P partial tiles of each block are added in wave order
// through LDS (double-buffered, one barrier per round); finer work units, so less tail at the end of a launch, for
// a barrier per round. Each wave has two steps in flight (the next step's loads are issued before this step's
// MFMAs, also across the barrier). The order of every sum depends on (K, WAVES, SHARE, split) only, so an output
// row does not depend on M (bitwise).
constexpr int kStageRow = 1024 + 16;   // staged weight row stride in LDS (bytes)
constexpr int kStageXMax = 2048;       // activation elements per row staged in LDS
constexpr int kStageXRow = kStageXMax + 8;

template <int KIND>
struct StagedStep {
  u32x4 w[16];

  __device__ __forceinline__ void load(const uint8_t* block, int64_t row_bytes, int64_t rows_left, int lane) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t rr = r < rows_left ? r : rows_left - 1;
      w[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(block + rr * row_bytes + lane * 16));
    }
  }
};

template <int KIND, int WAVES, bool SHARE>
__global__ __launch_bounds__(WAVES * kWave) void skinny_mfma_staged_kernel(const uint16_t* __restrict__ x,
                                                                           const uint8_t* __restrict__ w,
                                                                           const void* __restrict__ scale,
                                                                           int scale_dt, uint16_t* __restrict__ y,
                                                                           float* __restrict__ ws, int M, int64_t N,
                                                                           int64_t K, int split) {
  constexpr int kEB = KIND == kBf16 ? 2 : 1;
  constexpr int kStepK = 1024 / kEB;  // K elements per step (1 KiB of a weight row)
  constexpr int kMfmas = kStepK / 32; // MFMAs per step
  constexpr int kT = WAVES * kWave;
  __shared__ __attribute__((aligned(16))) uint8_t stage[WAVES][16 * kStageRow];
  __shared__ __attribute__((aligned(16))) uint16_t xs[16 * kStageXRow];
  __shared__ floatx4 red[SHARE ? 2 : 1][SHARE ? WAVES : 1][kWave];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int i = lane & 15;
  const int g = lane >> 4;
  const int sp = blockIdx.y;
  const int64_t kslice = K / split;
  const int64_t k_lo = sp * kslice;
  const int nsteps = static_cast<int>(kslice / kStepK);
  const int P = !SHARE ? 1 : nsteps < WAVES ? nsteps : WAVES;  // waves per block
  const int c = WAVES / P;                        // blocks per round
  const int Q = nsteps / P;                       // steps per wave and block
  const int jb = wave / P;
  const int p = wave % P;
  const int64_t nblocks = (N + 15) / 16;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * c;
  const int64_t per_round = static_cast<int64_t>(gridDim.x) * c;
  const int rounds = first < nblocks ? static_cast<int>((nblocks - first + per_round - 1) / per_round) : 0;
  const int units = rounds * Q;
  const int64_t row_bytes = K * kEB;
  uint8_t* st = stage[wave];

  // unit u of this wave: round u / Q, block (round * gridDim.x + blockIdx.x) * c + jb, step p + (u % Q) * P
  auto unit_block = [&](int u) { return (static_cast<int64_t>(u / Q) * gridDim.x + blockIdx.x) * c + jb; };
  auto issue = [&](StagedStep<KIND>& op, int u) {
    int64_t b = unit_block(u);
    if (b >= nblocks) b = nblocks - 1;  // a block past the end (last round): loads of the last block, never used
    const int s = p + (u % Q) * P;
    op.load(w + b * 16 * row_bytes + (k_lo + static_cast<int64_t>(s) * kStepK) * kEB, row_bytes, N - b * 16, lane);
  };

  StagedStep<KIND> buf[2];
  if (units > 0) issue(buf[0], 0);

  // the activations of the slice, after the first weight loads: xs[m][k] = x[m][k_lo + k] for m < M
  {
    const int cpr = static_cast<int>(kslice / 8);  // 16-byte chunks per row
    const int total = M * cpr;
    for (int e0 = 0; e0 < total; e0 += 8 * kT) {
      u32x4 v[8];
#pragma unroll
      for (int a = 0; a < 8; ++a) {
        const int e = e0 + a * kT + static_cast<int>(threadIdx.x);
        if (e < total)
          v[a] = *reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(e / cpr) * K + k_lo + 8 * (e % cpr));
      }
#pragma unroll
      for (int a = 0; a < 8; ++a) {
        const int e = e0 + a * kT + static_cast<int>(threadIdx.x);
        if (e < total) *reinterpret_cast<u32x4*>(&xs[(e / cpr) * kStageXRow + 8 * (e % cpr)]) = v[a];
      }
    }
  }
  __syncthreads();

  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
  auto process = [&](const StagedStep<KIND>& op, int u) {
    const int q = u % Q;
    const int64_t b = unit_block(u);
    if (b < nblocks) {
      const int s = p + q * P;
#pragma unroll
      for (int r = 0; r < 16; ++r) *reinterpret_cast<u32x4*>(&st[r * kStageRow + lane * 16]) = op.w[r];
#pragma unroll
      for (int jm = 0; jm < kMfmas; ++jm) {
        const int kx = s * kStepK + 32 * jm + 8 * g;
        const u32x4 bx = *reinterpret_cast<const u32x4*>(&xs[i * kStageXRow + kx]);
        u32x4 av;
        if constexpr (KIND == kBf16) {
          av = *reinterpret_cast<const u32x4*>(&st[i * kStageRow + 64 * jm + 16 * g]);
        } else {
          const uint2 qv = *reinterpret_cast<const uint2*>(&st[i * kStageRow + 32 * jm + 8 * g]);
          av = i8x8_to_bf16x8(qv.x, qv.y);
        }
        acc = mfma_bf16(av, bx, acc);
      }
    }
    if (q == Q - 1) {
      floatx4 t = acc;
      acc = floatx4{0.f, 0.f, 0.f, 0.f};
      if constexpr (SHARE) {
        const int buf_id = (u / Q) & 1;
        red[buf_id][wave][lane] = t;
        __syncthreads();
        if (p == 0) {
          t = red[buf_id][wave][lane];
          for (int o = 1; o < P; ++o) {
            const floatx4 v = red[buf_id][wave + o][lane];
            t.x += v.x;
            t.y += v.y;
            t.z += v.z;
            t.w += v.w;
          }
        }
      }
      if (p == 0 && b < nblocks) {
        const int m = lane & 15;
        if (m < M) {
          const float tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t n = b * 16 + 4 * g + r;
            if (n >= N) continue;
            float v = tv[r];
            if (split == 1) {
              if constexpr (KIND == kInt8) v *= load_scale(scale, n, scale_dt);
              y[static_cast<int64_t>(m) * N + n] = float_to_bf16_bits(v);
            } else {
              ws[(static_cast<int64_t>(sp) * M + m) * N + n] = v;
            }
          }
        }
      }
    }
  };

  for (int u = 0; u + 1 < units; u += 2) {
    issue(buf[1], u + 1);
    __builtin_amdgcn_sched_barrier(0);
    process(buf[0], u);
    issue(buf[0], u + 2 < units ? u + 2 : u);
    __builtin_amdgcn_sched_barrier(0);
    process(buf[1], u + 1);
  }
  if (units & 1) process(buf[0], units - 1);
}

}  // namespace

// The staged variant for (kind, waves, waves sharing each block), or null.
SkinnyFn mfma_staged_pick(int wkind, int waves, bool share) {
#define BP_STAGED(KIND)                                                                                  \
  switch (waves) {                                                                                       \
    case 1: return share ? &skinny_mfma_staged_kernel<KIND, 1, true> : &skinny_mfma_staged_kernel<KIND, 1, false>; \
    case 2: return share ? &skinny_mfma_staged_kernel<KIND, 2, true> : &skinny_mfma_staged_kernel<KIND, 2, false>; \
    case 4: return share ? &skinny_mfma_staged_kernel<KIND, 4, true> : &skinny_mfma_staged_kernel<KIND, 4, false>; \
    default: return nullptr;                                                                             \
  }
  if (wkind == kBf16) BP_STAGED(kBf16)
  if (wkind == kInt8) BP_STAGED(kInt8)
  return nullptr;
#undef BP_STAGED
}

int mfma_staged_k_max() { return kStageXMax; }

template <bool SILU>
SkinnyFn mfma_pick_t(int wkind, int rb, int waves, int depth) {
#define BP_MFMA_DEPTH(KIND, RB, W)                                     \
  switch (depth) {                                                     \
    case 1: return &skinny_mfma_kernel<KIND, RB, W, 1, SILU>;          \
    case 2: return &skinny_mfma_kernel<KIND, RB, W, 2, SILU>;          \
    default: return nullptr;                                           \
  }
#define BP_MFMA_WAVES(KIND, RB)                \
  switch (waves) {                             \
    case 1: BP_MFMA_DEPTH(KIND, RB, 1)         \
    case 2: BP_MFMA_DEPTH(KIND, RB, 2)         \
    case 4: BP_MFMA_DEPTH(KIND, RB, 4)         \
    case 8: BP_MFMA_DEPTH(KIND, RB, 8)         \
    default: return nullptr;                   \
  }
#define BP_MFMA_RB(KIND)                     \
  switch (rb) {                              \
    case 1: BP_MFMA_WAVES(KIND, 1)           \
    case 2: BP_MFMA_WAVES(KIND, 2)           \
    case 4: BP_MFMA_WAVES(KIND, 4)           \
    default: return nullptr;                 \
  }
  if (wkind == kBf16) BP_MFMA_RB(kBf16)
  if (wkind == kInt8) BP_MFMA_RB(kInt8)
  return nullptr;
#undef BP_MFMA_RB
#undef BP_MFMA_WAVES
#undef BP_MFMA_DEPTH
}

SkinnyFn mfma_pick(int wkind, int rb, int waves, int depth) { return mfma_pick_t<false>(wkind, rb, waves, depth); }

SkinnyFn mfma_silu_pick(int wkind, int rb, int waves, int depth) { return mfma_pick_t<true>(wkind, rb, waves, depth); }

int mfma_k_step(int wkind) { return wkind == kBf16 ? MfmaLayout<kBf16>::kStep : MfmaLayout<kInt8>::kStep; }

}  // namespace bp
