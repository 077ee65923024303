// The matrix-core skinny kernel (skinny_mf.h's operand layout) and its launch menu, shared by the translation units
// that instantiate it: skinny_mf.hip (any segment count per wave) and skinny_mf_n4 / n8 / n16.hip (launches whose
// waves have exactly 4, 8 or 16 K segments each, run as straight-line code). Every variant computes the same sums
// in the same order.
//
// Reference semantics: byteprof/optim/skinny.py:36-90 (kernel and _split_reduce), via skinny_mm
// (skinny.py:136-166).
#pragma once

#include <algorithm>

#include "byteprof_amd.h"
#include "skinny_mf.h"

namespace bp {

// Transform of the LDS-staged activation rows before the matmul (split 1: the workgroup holds whole rows).
struct MfPro {
  int kind;                  // 0 none, BP_PRO_UNIT_RMS, BP_PRO_NORM
  float eps;                 // BP_PRO_NORM: inside the root
  const uint16_t* gamma;     // BP_PRO_NORM: [K]
  const uint16_t* residual;  // BP_PRO_NORM: [M, K] or null
  uint16_t* xout;            // [M, K] or null: the transformed rows, written by workgroup (0, 0)
  int gl;                    // BP_PRO_NORM: 1 when gamma and the residual rows are staged in LDS (the launch sized it)
  const uint16_t* gamma2;    // BP_PRO_NORM: [K] or null: a second norm (no residual) of the transformed rows
  unsigned long long* tl;    // timeline builds (-DBP_TIMELINE): per-workgroup stamps [kMfTimelineWgs][8], or null
};

// Timeline builds: thread 0 of each workgroup (linear index below kMfTimelineWgs) stores s_memrealtime (100 MHz)
// at 0 entry, 1 the first segments' loads issued (after the activation staging, if any), 2 the first segment's
// MFMAs issued (its data arrived), 3 the last segment's MFMAs issued, 4 the waves' tiles in LDS (after the barrier),
// 5 the outputs stored, 6 the end. Normal builds compile none of it.
constexpr int kMfTimelineWgs = 16384;
#ifdef BP_TIMELINE
#define MF_TL(k)                                                        \
  do {                                                                  \
    if (threadIdx.x == 0) tl_[k] = __builtin_amdgcn_s_memrealtime();    \
  } while (0)
#else
#define MF_TL(k) \
  do {           \
  } while (0)
#endif

using MfFn = void (*)(const uint16_t*, const uint8_t*, const void*, int, uint16_t*, float*, int, int64_t, int64_t,
                      int, MfPro);

// The kernel of a launch whose waves have NSEG segments each (0: any count), or null when none is compiled; wr:
// row groups over the staged activations (1, or 2 / 4 with xl).
template <int NSEG>
MfFn mf_pick_n(int wkind, int mb, int rb, int waves, bool vec, int epi, bool xl, bool pro, int wr);

// In place, row by row:
//   BP_PRO_UNIT_RMS: x <- bf16(x * (1 / sqrt(mean(x^2)))) (an all-zero row is left as is);
//   BP_PRO_NORM:     x <- bf16(residual + bf16(gamma * (x * (1 / sqrt(mean(x^2) + eps))))) (no residual: the plain
//                    norm), and workgroup (0, 0) writes the rows to xout; with gamma2, then x <- bf16(gamma2 * (x *
//                    (1 / sqrt(mean(x^2) + eps)))) (a decoder's last post-feed-forward norm, then its final norm).
// The mean square is wave_sumsq's (common.h), the same bits whichever wave computes it, so the fused norm equals
// the separate norm launch (decode.hip, norm_residual_kernel) bit for bit. Wave w sums rows w, w + waves, ... into
// sums[] (LDS, one float per row); one barrier later every row is rewritten. gl (BP_PRO_NORM with pro.gl, else
// null): LDS copies of gamma [K], the residual rows [rows][K] and gamma2 [K] (if any), loaded ahead of the weights.
template <int NT>
__device__ void mf_prologue(uint16_t* xs, int rows, int K, MfPro pro, bool writer, const uint16_t* gl,
                            float* sums) {
  constexpr int kWaves = NT / kWave;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  for (int m = wave; m < rows; m += kWaves) {
    const float t = wave_sumsq_lds(xs + m * K, K);
    if ((threadIdx.x & (kWave - 1)) == 0) sums[m] = t;
  }
  __syncthreads();  // every row's sum is in sums[] before any row is rewritten
  for (int m = 0; m < rows; ++m) {
    uint16_t* row = xs + m * K;
    const float t = sums[m];
    if (pro.kind == BP_PRO_UNIT_RMS) {
      const float ms = t / static_cast<float>(K);
      const float inv = ms > 0.f ? 1.f / sqrtf(ms) : 1.f;
      for (int i = 4 * static_cast<int>(threadIdx.x); i < K; i += 4 * NT) {  // K is a multiple of 64
        const uint2 xq = *reinterpret_cast<const uint2*>(row + i);
        const uint32_t xw[4] = {xq.x << 16, xq.x & 0xffff0000u, xq.y << 16, xq.y & 0xffff0000u};
        uint32_t ov[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = float_to_bf16_bits(__uint_as_float(xw[e]) * inv);
        const uint2 o2{ov[0] | (ov[1] << 16), ov[2] | (ov[3] << 16)};
        *reinterpret_cast<uint2*>(row + i) = o2;
        if (writer && pro.xout != nullptr)
          *as_global_mut(reinterpret_cast<uint64_t*>(pro.xout + static_cast<int64_t>(m) * K + i)) =
              static_cast<uint64_t>(o2.x) | (static_cast<uint64_t>(o2.y) << 32);
      }
    } else {
      const float r = 1.f / sqrtf(t / static_cast<float>(K) + pro.eps);
      const bool has_res = pro.residual != nullptr;
      auto put = [&](int i, float g, float rv) {
        const float yv = round_to_bf16(g * (bf16_bits_to_float(row[i]) * r));
        const uint16_t v = float_to_bf16_bits(has_res ? rv + yv : yv);
        row[i] = v;
        if (writer && pro.xout != nullptr) as_global_mut(pro.xout)[static_cast<int64_t>(m) * K + i] = v;
      };
      if (gl != nullptr) {  // gamma and the residual rows in LDS: four elements per thread and step
        const uint16_t* gres = gl + (1 + m) * K;
        for (int i = 4 * static_cast<int>(threadIdx.x); i < K; i += 4 * NT) {
          const uint2 xq = *reinterpret_cast<const uint2*>(row + i);
          const uint2 gq = *reinterpret_cast<const uint2*>(gl + i);
          const uint2 rq = has_res ? *reinterpret_cast<const uint2*>(gres + i) : uint2{0u, 0u};
          const uint32_t xw[4] = {xq.x << 16, xq.x & 0xffff0000u, xq.y << 16, xq.y & 0xffff0000u};
          const uint32_t gw[4] = {gq.x << 16, gq.x & 0xffff0000u, gq.y << 16, gq.y & 0xffff0000u};
          const uint32_t rw[4] = {rq.x << 16, rq.x & 0xffff0000u, rq.y << 16, rq.y & 0xffff0000u};
          uint32_t ov[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float yv = round_to_bf16(__uint_as_float(gw[e]) * (__uint_as_float(xw[e]) * r));
            ov[e] = float_to_bf16_bits(has_res ? __uint_as_float(rw[e]) + yv : yv);
          }
          const uint2 o2{ov[0] | (ov[1] << 16), ov[2] | (ov[3] << 16)};
          *reinterpret_cast<uint2*>(row + i) = o2;
          if (writer && pro.xout != nullptr)
            *as_global_mut(reinterpret_cast<uint64_t*>(pro.xout + static_cast<int64_t>(m) * K + i)) =
                static_cast<uint64_t>(o2.x) | (static_cast<uint64_t>(o2.y) << 32);
        }
      } else {
        gptr<const uint16_t> gam = as_global(pro.gamma);
        gptr<const uint16_t> res = has_res ? as_global(pro.residual + static_cast<int64_t>(m) * K) : nullptr;
        for (int i = threadIdx.x; i < K; i += NT)
          put(i, bf16_bits_to_float(gam[i]), has_res ? bf16_bits_to_float(res[i]) : 0.f);
      }
    }
  }
  if (pro.kind == BP_PRO_NORM && pro.gamma2 != nullptr) {
    // the second norm: the same sums and roundings over the rewritten rows, gamma2 from LDS or memory
    __syncthreads();
    for (int m = wave; m < rows; m += kWaves) {
      const float t = wave_sumsq_lds(xs + m * K, K);
      if ((threadIdx.x & (kWave - 1)) == 0) sums[m] = t;
    }
    __syncthreads();
    const int nres = pro.residual != nullptr ? rows : 0;
    for (int m = 0; m < rows; ++m) {
      uint16_t* row = xs + m * K;
      const float r = 1.f / sqrtf(sums[m] / static_cast<float>(K) + pro.eps);
      if (gl != nullptr) {
        const uint16_t* g2 = gl + (1 + nres) * K;
        for (int i = 4 * static_cast<int>(threadIdx.x); i < K; i += 4 * NT) {
          const uint2 xq = *reinterpret_cast<const uint2*>(row + i);
          const uint2 gq = *reinterpret_cast<const uint2*>(g2 + i);
          const uint32_t xw[4] = {xq.x << 16, xq.x & 0xffff0000u, xq.y << 16, xq.y & 0xffff0000u};
          const uint32_t gw[4] = {gq.x << 16, gq.x & 0xffff0000u, gq.y << 16, gq.y & 0xffff0000u};
          uint32_t ov[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            ov[e] = float_to_bf16_bits(round_to_bf16(__uint_as_float(gw[e]) * (__uint_as_float(xw[e]) * r)));
          *reinterpret_cast<uint2*>(row + i) = uint2{ov[0] | (ov[1] << 16), ov[2] | (ov[3] << 16)};
        }
      } else {
        gptr<const uint16_t> g2 = as_global(pro.gamma2);
        for (int i = threadIdx.x; i < K; i += NT)
          row[i] = float_to_bf16_bits(round_to_bf16(bf16_bits_to_float(g2[i]) * (bf16_bits_to_float(row[i]) * r)));
      }
    }
  }
  __syncthreads();
}

#ifdef BP_MF_INSTANTIATE
namespace {

// EPI: 0 = y[m][n] (split 1) or fp32 partials ws[split][m][n]; 1 = the SiLU product of interleaved gate|up rows
// (rows 2f / 2f + 1 the gate / up rows of output f): y[m][f] = bf16(bf16(silu(bf16(g))) * bf16(u)).
// XL: the workgroup's activation rows and K range are staged in LDS (dynamic shared memory of
// min(M, 8 MB) x K-range x 2 bytes), their loads issued before the first weight loads; otherwise every segment's
// activation operand is loaded from memory with its weights. Same operands either way: the results are equal bit
// for bit. PRO (XL, split 1 only): a transform of the staged rows before the matmul (mf_prologue); for
// BP_PRO_NORM, gamma and the residual rows are loaded into LDS ahead of the weights too where the launch sized the
// LDS for them (pro.gl: 2 K (1 + rows) more bytes, always at one row, else within 80 KiB in all). NSEG > 0 (VEC only): every wave of the launch has exactly NSEG segments (the
// host checks K / (segment x split x waves) == NSEG), run as straight-line code (MfFixed); 0: any count (MfMain).
// WR > 1 (XL only, no prologue): WR row groups of 8 RB rows, each with its own WAVES waves splitting K as above, over
// the one LDS copy of the activation rows: the workgroup reads its activation operands once for 8 RB WR rows (the
// bytes per weight row fall by WR), every row's sum in the same order as with WR = 1.
template <int KIND, int MB, int RB, int WAVES, bool VEC, int EPI, bool XL, bool PRO, int NSEG, int WR = 1>
__global__ __launch_bounds__(WAVES * WR * kWave) void skinny_mf_kernel(const uint16_t* __restrict__ x,
                                                                  const uint8_t* __restrict__ w,
                                                                  const void* __restrict__ scale, int scale_dt,
                                                                  uint16_t* __restrict__ y, float* __restrict__ ws,
                                                                  int M, int64_t N, int64_t K, int split, MfPro pro) {
  using G = MfGeom<KIND>;
  static_assert(NSEG == 0 || VEC, "the fixed segment count needs vector loads");
  static_assert(WR == 1 || (XL && !PRO), "row groups share the staged activations (no prologue)");
  constexpr int NW = WAVES * WR;  // the workgroup's waves
  constexpr int NT = NW * kWave;
  constexpr int D = VEC ? mf_depth<KIND, MB, RB, !XL>() : 1;
  constexpr int kInFlight = NSEG > 0 && NSEG < D ? NSEG : D;  // weight segments issued before the staging commit
  __shared__ MfRed<WAVES, RB, MB> red[WR];
  __shared__ float pro_sums[PRO ? 8 * MB : 1];  // the prologue's per-row sums of squares
  extern __shared__ __attribute__((aligned(16))) uint16_t xs_lds[];

#ifdef BP_TIMELINE
  unsigned long long tl_[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const auto first = [&]() { MF_TL(2); };
#else
  const MfNoHook first;
#endif
  MF_TL(0);
  const int lane = threadIdx.x & (kWave - 1);
  // wave-uniform (a scalar value): the segment count below decides whether MFMAs run, and MFMAs ignore EXEC, so the
  // compiler must see those branches as uniform and make them scalar branches
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wk = WR == 1 ? wave : wave % WAVES;  // the wave's K share
  const int wr = WR == 1 ? 0 : wave / WAVES;     // its row group
  const MfLane ln(lane);
  constexpr int kRows = 8 * RB;       // a row group's rows
  constexpr int kRowsW = kRows * WR;  // the workgroup's rows
  const int64_t nw0 = static_cast<int64_t>(blockIdx.x) * kRowsW;
  const int64_t n0 = nw0 + wr * kRows;
  const int sp = blockIdx.y;
  // The epilogue's operands, ready before the weight stream. Left to the compiler, the output pointers' kernel-
  // argument loads sink into the epilogue and the int8 scales are loaded there: both then wait behind the
  // saturated weight stream (~1.3 us per workgroup, the tail of every launch). So y and ws are pinned in scalar
  // registers here, and an int8 launch at split 1 loads the scales of the rows this thread stores (every pass of
  // the epilogue loop gives thread t the workgroup's row t % 8RB WR, or rows 2 (t % 4RB WR) and + 1 with the SiLU
  // epilogue, as 8 RB WR divides the thread count) as raw halves, unconditionally (a 16-bit scale read twice).
  uint16_t* yk = y;
  float* wsk = ws;
  asm volatile("" : "+s"(yk), "+s"(wsk));
  uint32_t sraw[EPI == 0 ? 1 : 2][2];
  if constexpr (KIND == kInt8) {
    // unconditional loads (a conditional one would be waited for where the branches meet); without scales to read
    // (split > 1: the reduce applies them; the partials launch passes none) they read x[0], unused
    const bool have = split == 1 && scale != nullptr;
    const int rr0 =
        EPI == 0 ? static_cast<int>(threadIdx.x % kRowsW) : 2 * static_cast<int>(threadIdx.x % (kRowsW / 2));
    const bool f32 = scale_dt == BP_DT_F32;
    const auto p = as_global(have ? static_cast<const uint16_t*>(scale) : x);
#pragma unroll
    for (int u = 0; u < (EPI == 0 ? 1 : 2); ++u) {
      const int64_t n = std::min<int64_t>(nw0 + rr0 + u, N - 1);
      const int64_t e = !have ? 0 : f32 ? 2 * n : n;
      sraw[u][0] = p[e];
      sraw[u][1] = p[e + (have && f32 ? 1 : 0)];
    }
  }
  // the prefetched scale of the thread's row u
  const auto row_scale = [&](int u) -> float {
    if (scale_dt == BP_DT_F32) return __uint_as_float(sraw[u][0] | (sraw[u][1] << 16));
    if (scale_dt == BP_DT_BF16) return bf16_bits_to_float(sraw[u][0]);
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(sraw[u][0])));
  };
  const int64_t nseg_all = (K + G::kSeg - 1) / G::kSeg;
  // split 1 (every decode-step launch) needs no division
  const int64_t s_lo = split == 1 ? 0 : sp * nseg_all / split;
  const int64_t s_hi = split == 1 ? nseg_all : (sp + 1) * nseg_all / split;
  const int64_t s_first = s_lo + wk;
  const int64_t nseg = NSEG > 0 ? NSEG : mf_uniform(s_first < s_hi ? (s_hi - s_first + WAVES - 1) / WAVES : 0);

  // the lane's weight rows (rows past N read row N - 1; their outputs are never stored), advanced to the lane's
  // 16 bytes of a segment (VEC = false: the row start; the element loads add the lane's K offset kl)
  const int64_t kl = static_cast<int64_t>(G::kLaneK) * ln.slot();
  const uint8_t* wrow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int64_t row = std::min<int64_t>(n0 + 8 * rb + ln.r, N - 1);
    wrow[rb] = w + row * K * G::kEB + (VEC ? 16 * ln.slot() : 0);
  }
  floatx4 acc[RB][MB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[rb][b] = floatx4{0.f, 0.f, 0.f, 0.f};

  if constexpr (XL) {
    constexpr int kNT = NT;
    constexpr int kPer = 4;
    const int mrows = M < 8 * MB ? M : 8 * MB;
    const int kn = static_cast<int>((s_hi - s_lo) * G::kSeg);
    const int64_t k_lo = s_lo * G::kSeg;
    const int passes = (mrows * (kn / 8) + kPer * kNT - 1) / (kPer * kNT);
    MfStage<kNT, kPer> stage;
    stage.issue(x, mrows, K, k_lo, kn, 0);  // ahead of the weight loads: the commit waits for these only
    MfXLds<KIND, MB> xs;
    xs.init(xs_lds, mrows, kn, k_lo, ln);
    // BP_PRO_NORM with pro.gl: gamma and the residual rows straight into LDS after the staged rows (64 lanes x 16
    // bytes per load, no registers held), ahead of the weight loads
    const uint16_t* gl = nullptr;
    if constexpr (PRO) {
      // rows past the register pass (kPer pieces per thread): straight into LDS, 64 pieces of 16 bytes per load
      // (piece e at element 8 e of the staged rows), ahead of the weight loads as well
      const int pieces = mrows * (kn / 8);
      for (int c = kPer * NW + wave; c * kWave < pieces; c += NW) {
        const int e = c * kWave + lane;
        if (e < pieces)
          __builtin_amdgcn_global_load_lds(
              as_global(x + static_cast<int64_t>(e / (kn / 8)) * K + k_lo + 8 * (e % (kn / 8))),
              (__attribute__((address_space(3))) void*)(xs_lds + c * 512), 16, 0, 0);
      }
      if (pro.kind == BP_PRO_NORM && pro.gl) {
        uint16_t* dst = xs_lds + mrows * kn;
        gl = dst;
        // LDS: gamma [kn], then the residual rows [kn] each
        if (mrows == 1) {
          uint16_t* dst2 = dst + (pro.residual != nullptr ? 2 : 1) * kn;  // gamma2 after gamma and the residual
          for (int j = wave; j * 512 < kn; j += NW) {
            const int e = j * 512 + 8 * lane;
            if (e < kn) {
              __builtin_amdgcn_global_load_lds(as_global(pro.gamma + e),
                                               (__attribute__((address_space(3))) void*)(dst + j * 512), 16, 0, 0);
              if (pro.residual != nullptr)
                __builtin_amdgcn_global_load_lds(as_global(pro.residual + e),
                                                 (__attribute__((address_space(3))) void*)(dst + kn + j * 512), 16,
                                                 0, 0);
              if (pro.gamma2 != nullptr)
                __builtin_amdgcn_global_load_lds(as_global(pro.gamma2 + e),
                                                 (__attribute__((address_space(3))) void*)(dst2 + j * 512), 16, 0, 0);
            }
          }
        } else {
          const int nres = pro.residual != nullptr ? mrows : 0;
          for (int j = wave; j * 512 < kn; j += NW) {
            const int e = j * 512 + 8 * lane;
            if (e < kn) {
              __builtin_amdgcn_global_load_lds(as_global(pro.gamma + e),
                                               (__attribute__((address_space(3))) void*)(dst + j * 512), 16, 0, 0);
              for (int r = 0; r < nres; ++r)
                __builtin_amdgcn_global_load_lds(
                    as_global(pro.residual + static_cast<int64_t>(r) * K + e),
                    (__attribute__((address_space(3))) void*)(dst + (1 + r) * kn + j * 512), 16, 0, 0);
              if (pro.gamma2 != nullptr)
                __builtin_amdgcn_global_load_lds(as_global(pro.gamma2 + e),
                                                 (__attribute__((address_space(3))) void*)(dst + (1 + nres) * kn +
                                                                                           j * 512),
                                                 16, 0, 0);
            }
          }
        }
      }
    }
    // The staged rows (and the prologue's operands) were loaded before the kInFlight x RB weight loads: waiting for them
    // leaves the weights in flight. The prologue variants stage their first pass through registers and the rest by
    // the LDS loads above, all before the weights, so the transform runs while the weights stream in.
    auto commit = [&]() {
      mf_wait_vm<kInFlight * RB>();
      stage.commit(xs_lds, mrows, kn, 0);
      if constexpr (PRO) {
        __syncthreads();
        if (pro.kind != 0)
          mf_prologue<kNT>(xs_lds, mrows, kn, pro, blockIdx.x == 0 && blockIdx.y == 0, gl, pro_sums);
      } else {
        for (int pass = 1; pass < passes; ++pass) {
          stage.issue(x, mrows, K, k_lo, kn, pass);
          stage.commit(xs_lds, mrows, kn, pass);
        }
        __syncthreads();
      }
      MF_TL(1);
    };
    if constexpr (NSEG > 0)
      MfFixed<KIND, MB, RB, D, NSEG, false, MfXLds<KIND, MB>>::run(wrow, xs, s_first, WAVES, acc, commit, first);
    else
      MfMain<KIND, MB, RB, D, true, false, MfXLds<KIND, MB>>::run(wrow, xs, x, K, kl, s_first, WAVES, nseg, acc,
                                                                 commit, first);
  } else if constexpr (VEC) {
    MfXGlobal<KIND, MB, true> xs;
    xs.init(x, M, K, ln);
    const auto issued = [&]() { MF_TL(1); };
    if constexpr (NSEG > 0)
      MfFixed<KIND, MB, RB, D, NSEG, true, MfXGlobal<KIND, MB, true>>::run(wrow, xs, s_first, WAVES, acc, issued,
                                                                           first);
    else
      MfMain<KIND, MB, RB, D, true, true, MfXGlobal<KIND, MB, true>>::run(wrow, xs, x, K, kl, s_first, WAVES, nseg,
                                                                          acc, issued, first);
  } else {
    // element loads with bounds (K not a multiple of the segment or unaligned operands): same segments, same order
    MfXGlobal<KIND, MB, false> xs;
    xs.init(x, M, K, ln);
    MfMain<KIND, MB, RB, 1, false, true, MfXGlobal<KIND, MB, false>>::run(wrow, xs, x, K, kl, s_first, WAVES, nseg,
                                                                          acc);
  }
  MF_TL(3);
  mf_fold_halves<RB, MB>(acc);
  mf_store_red<WAVES, RB, MB>(red[wr], acc, wk, lane);
  __syncthreads();
  MF_TL(4);

  if constexpr (EPI == 0) {
    const int cols = M < 8 * MB ? M : 8 * MB;
    for (int e = threadIdx.x; e < kRowsW * cols; e += NT) {
      const int m = e / kRowsW;
      const int rw = e % kRowsW;  // the workgroup's row: row group rw / 8RB, row rw % 8RB of it
      const int64_t n = nw0 + rw;
      if (n >= N) continue;
      float t = mf_total<WAVES, RB, MB>(red[rw / kRows], rw % kRows, m);
      if (split == 1) {
        if constexpr (KIND == kInt8) t *= row_scale(0);
        yk[static_cast<int64_t>(m) * N + n] = float_to_bf16_bits(t);
      } else {
        wsk[(static_cast<int64_t>(sp) * M + m) * N + n] = t;
      }
    }
  } else {
    const int cols = M < 8 * MB ? M : 8 * MB;
    for (int e = threadIdx.x; e < (kRowsW / 2) * cols; e += NT) {
      const int m = e / (kRowsW / 2);
      const int rw = 2 * (e % (kRowsW / 2));
      const int64_t n = nw0 + rw;  // the gate row; n + 1 the up row
      if (n + 1 >= N) continue;
      float gv = mf_total<WAVES, RB, MB>(red[rw / kRows], rw % kRows, m);
      float uv = mf_total<WAVES, RB, MB>(red[rw / kRows], rw % kRows + 1, m);
      if constexpr (KIND == kInt8) {
        gv *= row_scale(0);
        uv *= row_scale(EPI == 0 ? 0 : 1);
      }
      const float gb = round_to_bf16(gv);
      const float a = round_to_bf16(gb / (1.f + expf(-gb)));
      yk[static_cast<int64_t>(m) * (N / 2) + n / 2] = float_to_bf16_bits(a * round_to_bf16(uv));
    }
  }
  MF_TL(5);
#ifdef BP_TIMELINE
  __builtin_amdgcn_s_waitcnt(0);  // the stores done
  MF_TL(6);
  const int64_t wg = static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
  if (threadIdx.x == 0 && pro.tl != nullptr && wg < kMfTimelineWgs)
    for (int e = 0; e < 8; ++e) pro.tl[wg * 8 + e] = tl_[e];
#endif
}


// Compiled menu: activation blocks MB in {1, 2, 4, 8} (M <= 8, 16, 32, 64) x row blocks RB in {1, 2, 4} (RB 4 up
// to MB 2) x waves in {1, 2, 4, 8}; the SiLU epilogue and the LDS-staged activations up to MB 2; the element-load
// variant at RB 1, 4 waves.
template <int NSEG, int KIND, int MB, int RB, int EPI, bool XL, bool PRO>
MfFn pick_waves(int waves) {
  switch (waves) {
    case 1: return &skinny_mf_kernel<KIND, MB, RB, 1, true, EPI, XL, PRO, NSEG>;
    case 2: return &skinny_mf_kernel<KIND, MB, RB, 2, true, EPI, XL, PRO, NSEG>;
    case 4: return &skinny_mf_kernel<KIND, MB, RB, 4, true, EPI, XL, PRO, NSEG>;
    case 8: return &skinny_mf_kernel<KIND, MB, RB, 8, true, EPI, XL, PRO, NSEG>;
    default: return nullptr;
  }
}

template <int NSEG, int KIND, int MB, int EPI, bool XL, bool PRO = false>
MfFn pick_rb(int rb, int waves) {
  switch (rb) {
    case 1: return pick_waves<NSEG, KIND, MB, 1, EPI, XL, PRO>(waves);
    case 2: return pick_waves<NSEG, KIND, MB, 2, EPI, XL, PRO>(waves);
    case 4:
      if constexpr (MB <= 2) return pick_waves<NSEG, KIND, MB, 4, EPI, XL, PRO>(waves);
      return nullptr;
    default: return nullptr;
  }
}

template <int NSEG, int KIND, int EPI, bool XL>
MfFn pick_mb(int mb, int rb, int waves, bool vec) {
  if (!vec) {
    if constexpr (EPI == 0 && !XL && NSEG == 0) {
      if (waves != 4) return nullptr;
      switch (mb) {
        case 1: return &skinny_mf_kernel<KIND, 1, 1, 4, false, 0, false, false, 0>;
        case 2: return &skinny_mf_kernel<KIND, 2, 1, 4, false, 0, false, false, 0>;
        case 4: return &skinny_mf_kernel<KIND, 4, 1, 4, false, 0, false, false, 0>;
        case 8: return &skinny_mf_kernel<KIND, 8, 1, 4, false, 0, false, false, 0>;
        default: return nullptr;
      }
    }
    return nullptr;
  }
  switch (mb) {
    case 1: return pick_rb<NSEG, KIND, 1, EPI, XL>(rb, waves);
    case 2: return pick_rb<NSEG, KIND, 2, EPI, XL>(rb, waves);
    case 4:
      if constexpr (EPI == 0 && !XL) return pick_rb<NSEG, KIND, 4, EPI, XL>(rb, waves);
      return nullptr;
    case 8:
      if constexpr (EPI == 0 && !XL) return pick_rb<NSEG, KIND, 8, EPI, XL>(rb, waves);
      return nullptr;
    default: return nullptr;
  }
}

// The prologue variants: staged activations, up to 16 rows, both epilogues.
template <int NSEG, int KIND, int EPI>
MfFn pick_pro(int mb, int rb, int waves) {
  switch (mb) {
    case 1: return pick_rb<NSEG, KIND, 1, EPI, true, true>(rb, waves);
    case 2: return pick_rb<NSEG, KIND, 2, EPI, true, true>(rb, waves);
    default: return nullptr;
  }
}

// Row groups (WR 2 / 4): the staged-activation kernels at 9..16 rows (MB 2), both epilogues, waves x WR <= 16.
template <int NSEG, int KIND, int RB, int EPI, int WR>
MfFn pick_wr_waves(int waves) {
  switch (waves) {
    case 2: return &skinny_mf_kernel<KIND, 2, RB, 2, true, EPI, true, false, NSEG, WR>;
    case 4: return &skinny_mf_kernel<KIND, 2, RB, 4, true, EPI, true, false, NSEG, WR>;
    case 8:
      if constexpr (WR == 2) return &skinny_mf_kernel<KIND, 2, RB, 8, true, EPI, true, false, NSEG, WR>;
      return nullptr;
    default: return nullptr;
  }
}

template <int NSEG, int KIND, int EPI, int WR>
MfFn pick_wr_rb(int rb, int waves) {
  switch (rb) {
    case 1: return pick_wr_waves<NSEG, KIND, 1, EPI, WR>(waves);
    case 2: return pick_wr_waves<NSEG, KIND, 2, EPI, WR>(waves);
    case 4: return pick_wr_waves<NSEG, KIND, 4, EPI, WR>(waves);
    default: return nullptr;
  }
}

template <int NSEG, int KIND>
MfFn mf_pick_kind(int mb, int rb, int waves, bool vec, int epi, bool xl, bool pro, int wr) {
  if (NSEG > 0 && !vec) return nullptr;
  if (wr != 1) {
    if constexpr (NSEG == 16) {
      return nullptr;  // K ranges of 16 segments a wave do not stage at 16 rows
    } else {
      if (!vec || !xl || pro || mb != 2 || (wr != 2 && wr != 4)) return nullptr;
      if (epi == 0) return wr == 2 ? pick_wr_rb<NSEG, KIND, 0, 2>(rb, waves) : pick_wr_rb<NSEG, KIND, 0, 4>(rb, waves);
      return wr == 2 ? pick_wr_rb<NSEG, KIND, 1, 2>(rb, waves) : pick_wr_rb<NSEG, KIND, 1, 4>(rb, waves);
    }
  }
  if (pro)
    return vec && xl ? (epi == 0 ? pick_pro<NSEG, KIND, 0>(mb, rb, waves) : pick_pro<NSEG, KIND, 1>(mb, rb, waves))
                     : nullptr;
  if (epi == 0)
    return xl ? pick_mb<NSEG, KIND, 0, true>(mb, rb, waves, vec) : pick_mb<NSEG, KIND, 0, false>(mb, rb, waves, vec);
  return xl ? pick_mb<NSEG, KIND, 1, true>(mb, rb, waves, vec) : pick_mb<NSEG, KIND, 1, false>(mb, rb, waves, vec);
}

}  // namespace

template <int NSEG>
MfFn mf_pick_n(int wkind, int mb, int rb, int waves, bool vec, int epi, bool xl, bool pro, int wr) {
  if (wkind == kBf16) return mf_pick_kind<NSEG, kBf16>(mb, rb, waves, vec, epi, xl, pro, wr);
  if (wkind == kInt8) return mf_pick_kind<NSEG, kInt8>(mb, rb, waves, vec, epi, xl, pro, wr);
  return nullptr;
}

#endif  // BP_MF_INSTANTIATE

}  // namespace bp
