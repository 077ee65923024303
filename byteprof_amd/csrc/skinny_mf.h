// Skinny weight-only matmul on the matrix cores with a streaming-friendly operand layout, gfx950:
// y[M, N] = x[M, K] . W[N, K]^T for 1..64 activation rows, bf16 activations, fp32 accumulation; weights bf16, or
// int8 with one scale per output row (converted exactly to bf16 in registers; the scale multiplies the fp32 sum).
//
// Operand layout (v_mfma_f32_16x16x32_bf16: A 16 x 32, B 32 x 16, D 16 x 16; lane l holds A row l % 16 and B column
// l % 16 at K slots 8 (l / 16) .. + 7, and D rows 4 (l / 16) .. + 3 of column l % 16):
//   - a row block is 8 consecutive weight rows; a K segment is 128 bytes of each row (64 bf16 / 128 int8 weights);
//   - one 16-byte load per lane reads a whole segment of a block: lane (g = l / 16, i = l % 16) reads bytes
//     16 (2 g + h) .. + 15 of row i % 8, h = i / 8, so each row is one full 128-byte line per load instruction (the
//     rate of 1 KiB-per-row streaming; 16 rows x 64 bytes per instruction streams ~40% slower);
//   - A row i of the MFMA is then weight row i % 8 restricted to half h of the segment's K slots, and B column j is
//     activation row 8 b + j % 8 (b: the 8-row activation block) restricted to half j / 8; the lane's A and B slots
//     cover the same K indices, so D[i][j] is a partial dot product exactly when i / 8 == j / 8: D[r][m] (half 0)
//     plus D[r + 8][m + 8] (half 1) is the segment's contribution to output (row r, activation row m);
//   - bf16: one MFMA per load and activation block; int8: the 16 loaded bytes are two MFMA A operands (bytes 0-7,
//     8-15), the activation operand likewise.
// Work: a workgroup owns RB row blocks and WAVES wavefronts; segment s of the workgroup's K range [s_lo, s_hi) goes
// to wave (s - s_lo) % WAVES; each wave keeps D segments in flight; the wave's tiles are combined over the two halves
// in registers (half 0 + half 1), then over the waves in LDS in wave order; with split > 1 the K ranges of grid.y
// store fp32 partials that a second kernel adds in split order.
// The order of every sum depends on (K, WAVES, split) only: output row m is bitwise independent of M, of RB, of the
// activation-block count and of which kernel (plain, grouped, chained) computes it.
//
// Reference semantics: byteprof/optim/skinny.py:36-90 (the kernel's bf16 / int8 modes and split reduce), via
// skinny_mm (skinny.py:136-166) for every activation row count up to MAX_M = 64 (skinny.py:32).
#pragma once

#include "common.h"

namespace bp {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int KIND>
struct MfGeom {
  static constexpr int kEB = KIND == kBf16 ? 2 : 1;        // bytes per weight
  static constexpr int kSeg = 128 / kEB;                   // K elements of a row per segment
  static constexpr int kLaneK = 16 / kEB;                  // K elements a lane loads per segment
  static constexpr int kParts = KIND == kBf16 ? 1 : 2;     // MFMA operands per lane per segment
};

// Lane roles shared by weight and activation operands.
struct MfLane {
  int g, i, h, r;
  __device__ __forceinline__ explicit MfLane(int lane) : g(lane >> 4), i(lane & 15), h((lane & 15) >> 3),
                                                         r(lane & 7) {}
  __device__ __forceinline__ int slot() const { return 2 * g + h; }  // 16-byte piece of the segment
};

__device__ __forceinline__ floatx4 mf_mfma(u32x4 a, u32x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// Eight int8 weights (two dwords) as eight bf16 values (exact).
__device__ __forceinline__ u32x4 mf_i8x8(uint32_t d0, uint32_t d1) {
  return u32x4{i8pair_to_bf16x2(d0, 0), i8pair_to_bf16x2(d0, 16), i8pair_to_bf16x2(d1, 0), i8pair_to_bf16x2(d1, 16)};
}

// 8 bf16 activations x_row[k .. k + 7] (zeros past K); VEC: one aligned 16-byte load.
template <bool VEC>
__device__ __forceinline__ u32x4 mf_load_x8(const uint16_t* __restrict__ xrow, int64_t k, int64_t K) {
  if constexpr (VEC) {
    return *reinterpret_cast<const u32x4*>(xrow + k);
  } else {
    uint32_t d[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = k + 2 * j < K ? xrow[k + 2 * j] : 0u;
      const uint32_t hi = k + 2 * j + 1 < K ? xrow[k + 2 * j + 1] : 0u;
      d[j] = lo | (hi << 16);
    }
    return u32x4{d[0], d[1], d[2], d[3]};
  }
}

// The lane's 16 weight bytes of row `wrow` at element k (zeros past K); VEC: one aligned non-temporal load.
template <int KIND, bool VEC>
__device__ __forceinline__ u32x4 mf_load_w16(const uint8_t* __restrict__ wrow, int64_t k, int64_t K) {
  using G = MfGeom<KIND>;
  if constexpr (VEC) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + k * G::kEB));
  } else {
    uint32_t d[4] = {0u, 0u, 0u, 0u};
    if constexpr (KIND == kBf16) {
      const uint16_t* p = reinterpret_cast<const uint16_t*>(wrow);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (k + e < K) d[e >> 1] |= static_cast<uint32_t>(p[k + e]) << (16 * (e & 1));
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (k + e < K) d[e >> 2] |= static_cast<uint32_t>(wrow[k + e]) << (8 * (e & 3));
    }
    return u32x4{d[0], d[1], d[2], d[3]};
  }
}

// Activation operands read from global memory (rows past M read row 0; their columns are never stored).
template <int KIND, int MB, bool VEC>
struct MfXGlobal {
  using G = MfGeom<KIND>;
  const uint16_t* row[MB];  // the lane's activation row, advanced to the lane's K offset
  int64_t kl;               // the lane's K offset within a segment
  int64_t K;

  __device__ __forceinline__ void init(const uint16_t* __restrict__ x, int M, int64_t K_, const MfLane& ln) {
    K = K_;
    kl = static_cast<int64_t>(G::kLaneK) * ln.slot();
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const int m = 8 * b + ln.r;
      row[b] = x + static_cast<int64_t>(m < M ? m : 0) * K;
    }
  }
  // operand `part` of segment s for activation block b
  __device__ __forceinline__ u32x4 load(int64_t s, int b, int part) const {
    return mf_load_x8<VEC>(row[b], s * G::kSeg + kl + 8 * part, K);
  }
};

// The vector form: one buffer resource over the M x K activations (the launch takes it for K < 2^24: with up to 64
// rows, 2 M K < 2^31 bytes).
// A lane of a row past M has an offset past the resource, so its loads return zeros without a memory request:
// the padding rows of the last activation block (7 of 8 at 9 rows) cost no memory traffic.
template <int KIND, int MB>
struct MfXGlobal<KIND, MB, true> {
  using G = MfGeom<KIND>;
  static constexpr uint32_t kPast = 0x80000000u;  // beyond any resource: 2 M K < 2^31
  __amdgpu_buffer_rsrc_t rs;
  uint32_t off[MB];  // byte offset of the lane's row at its K offset within a segment, or kPast

  __device__ __forceinline__ void init(const uint16_t* __restrict__ x, int M, int64_t K, const MfLane& ln) {
    rs = buffer_rsrc(x, static_cast<int>(2 * M * K));
    const int64_t kl = static_cast<int64_t>(G::kLaneK) * ln.slot();
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const int m = 8 * b + ln.r;
      off[b] = m < M ? static_cast<uint32_t>(2 * (m * K + kl)) : kPast;
    }
  }
  __device__ __forceinline__ u32x4 load(int64_t s, int b, int part) const {
    const uint32_t o = off[b] + static_cast<uint32_t>(2 * (s * G::kSeg + 8 * part));
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0));
  }
};

// Activation operands read from an LDS copy xs[m][k] of the workgroup's activation rows (row stride `stride`
// elements; segment s at element s * kSeg - k_base; rows past M read row 0 of the copy, never stored).
template <int KIND, int MB>
struct MfXLds {
  using G = MfGeom<KIND>;
  const uint16_t* row[MB];
  __device__ __forceinline__ void init(const uint16_t* xs, int M, int stride, int64_t k_base, const MfLane& ln) {
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const int m = 8 * b + ln.r;
      row[b] = xs + static_cast<int64_t>(m < M ? m : 0) * stride + G::kLaneK * ln.slot() - k_base;
    }
  }
  __device__ __forceinline__ u32x4 load(int64_t s, int b, int part) const {
    return *reinterpret_cast<const u32x4*>(row[b] + s * G::kSeg + 8 * part);
  }
};

// Copies x[m][k_lo .. k_lo + kn) for m < M into LDS xs[m][0 .. kn) (16-byte pieces, all threads of the workgroup).
// The global loads of a pass are issued before anything else waits, so a caller that issued them ahead of its
// weight loads (stage_issue, then weight loads, then stage_commit) only waits for these loads, not the weights'.
template <int NT, int PER>
struct MfStage {
  u32x4 v[PER];
  __device__ __forceinline__ void issue(const uint16_t* __restrict__ x, int M, int64_t K, int64_t k_lo, int kn,
                                        int pass) {
    const int pieces = M * (kn / 8);
#pragma unroll
    for (int a = 0; a < PER; ++a) {
      const int e = (pass * PER + a) * NT + static_cast<int>(threadIdx.x);
      if (e < pieces)
        v[a] = *reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(e / (kn / 8)) * K + k_lo + 8 * (e % (kn / 8)));
    }
  }
  __device__ __forceinline__ void commit(uint16_t* xs, int M, int kn, int pass) const {
    const int pieces = M * (kn / 8);
#pragma unroll
    for (int a = 0; a < PER; ++a) {
      const int e = (pass * PER + a) * NT + static_cast<int>(threadIdx.x);
      if (e < pieces) *reinterpret_cast<u32x4*>(xs + (e / (kn / 8)) * kn + 8 * (e % (kn / 8))) = v[a];
    }
  }
};

// s_waitcnt for at most N outstanding vector-memory loads of the wave, no wait on the other counters (gfx9
// encoding: vmcnt in bits 3:0 and 15:14, expcnt in 6:4, lgkmcnt in 11:8). Loads complete in issue order, so after
// mf_wait_vm<N>() every load but the last N issued has completed.
template <int N>
__device__ __forceinline__ void mf_wait_vm() {
  constexpr int n = N > 63 ? 63 : N;
  __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// No-op hook of MfMain::run.
struct MfNoHook {
  __device__ __forceinline__ void operator()() const {}
};

// The segments of one wave, D in flight. XS: MfXGlobal (x from memory, loaded with the weights) or MfXLds (x staged
// in LDS). acc[rb][b]: the wave's 16 x 16 tile of row block rb and activation block b. Segment idx of the wave is
// s_first + idx * stride; `ph` is an in-bounds, cached address that the loads of placeholder steps past the wave's
// last segment read (every iteration issues the same loads, so the compiler's wait counts stay exact). `hook` runs
// after the first D segments' loads are issued and before the first MFMA (the LDS staging of the activations).
// nseg must be wave-uniform: it decides whether MFMAs run, and MFMAs ignore EXEC.
template <int KIND, int MB, int RB, int D, bool VEC, bool XMEM, class XS>
struct MfMain {
  using G = MfGeom<KIND>;
  static constexpr int kXP = XMEM ? MB * G::kParts : 1;  // activation operands carried per slot
  struct Slot {
    u32x4 w[RB];
    u32x4 x[kXP];
  };

  // The loads of segment s into a slot (vector loads; wrow[rb] advanced to the lane's bytes of a segment).
  __device__ __forceinline__ static void load_slot(Slot& sl, const uint8_t* const (&wrow)[RB], const XS& xs,
                                                   int64_t s) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      sl.w[rb] = __builtin_nontemporal_load(as_global(reinterpret_cast<const u32x4*>(wrow[rb] + s * 128)));
    if constexpr (XMEM) {
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int p = 0; p < G::kParts; ++p) sl.x[b * G::kParts + p] = xs.load(s, b, p);
    }
  }

  // The MFMAs of segment s (its weights in the slot) into the wave's tiles.
  __device__ __forceinline__ static void compute_slot(const Slot& sl, const XS& xs, int64_t s,
                                                      floatx4 (&acc)[RB][MB]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      u32x4 a[G::kParts];
      if constexpr (KIND == kBf16) {
        a[0] = sl.w[rb];
      } else {
        a[0] = mf_i8x8(sl.w[rb].x, sl.w[rb].y);
        a[1] = mf_i8x8(sl.w[rb].z, sl.w[rb].w);
      }
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int p = 0; p < G::kParts; ++p) {
          u32x4 bx;
          if constexpr (XMEM) {
            bx = sl.x[b * G::kParts + p];
          } else {
            bx = xs.load(s, b, p);
          }
          acc[rb][b] = mf_mfma(a[p], bx, acc[rb][b]);
        }
    }
  }

  // wrow[rb]: the lane's weight row of block rb, advanced to the lane's byte offset in a segment.
  // (VEC = false: wrow[rb] is the row start and kl the lane's K offset in a segment, for bounded element loads.)
  template <class Hook = MfNoHook, class First = MfNoHook>
  __device__ __forceinline__ static void run(const uint8_t* const (&wrow)[RB], const XS& xs, const void* ph,
                                             int64_t K, int64_t kl, int64_t s_first, int64_t stride, int64_t nseg,
                                             floatx4 (&acc)[RB][MB], const Hook& hook = Hook(),
                                             const First& first = First()) {
    Slot buf[D];
    auto issue = [&](Slot& sl, int64_t idx) {
      const bool live = idx < nseg;
      const int64_t s = s_first + (live ? idx : 0) * stride;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        if constexpr (VEC) {
          const uint8_t* p = live ? wrow[rb] + s * 128 : static_cast<const uint8_t*>(ph);
          sl.w[rb] = __builtin_nontemporal_load(as_global(reinterpret_cast<const u32x4*>(p)));
        } else {
          sl.w[rb] = live ? mf_load_w16<KIND, false>(wrow[rb], s * G::kSeg + kl, K) : u32x4{0u, 0u, 0u, 0u};
        }
      }
      if constexpr (XMEM) {
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
          for (int p = 0; p < G::kParts; ++p) sl.x[b * G::kParts + p] = xs.load(s, b, p);
      }
    };
#pragma unroll
    for (int d = 0; d < D; ++d) issue(buf[d], d);
    hook();
    for (int64_t base = 0; base < nseg; base += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        if (base + d < nseg) compute_slot(buf[d], xs, s_first + (base + d) * stride, acc);
        if (d == 0 && base == 0) first();
        issue(buf[d], base + d + D);
      }
    }
  }
};

// The segments of one wave when their count NSEG is a compile-time constant (every wave of the launch has exactly
// NSEG): straight-line code, D in flight, no load past the wave's last segment, so the compiler's wait counts are
// exact and the wave ends as soon as its last MFMA is issued. Same segments, same order and same MFMA chain as
// MfMain::run (bitwise equal results). `hook` runs after the first min(D, NSEG) segments' loads are issued.
template <int KIND, int MB, int RB, int D, int NSEG, bool XMEM, class XS>
struct MfFixed {
  using Ops = MfMain<KIND, MB, RB, 1, true, XMEM, XS>;
  static constexpr int kD = D < NSEG ? D : NSEG;  // segments in flight

  template <class Hook = MfNoHook, class First = MfNoHook>
  __device__ __forceinline__ static void run(const uint8_t* const (&wrow)[RB], const XS& xs, int64_t s_first,
                                             int64_t stride, floatx4 (&acc)[RB][MB], const Hook& hook = Hook(),
                                             const First& first = First()) {
    typename Ops::Slot buf[kD];
#pragma unroll
    for (int i = 0; i < kD; ++i) Ops::load_slot(buf[i], wrow, xs, s_first + i * stride);
    hook();
#pragma unroll
    for (int i = 0; i < NSEG; ++i) {
      Ops::compute_slot(buf[i % kD], xs, s_first + i * stride, acc);
      if (i == 0) first();
      if (i + kD < NSEG) Ops::load_slot(buf[i % kD], wrow, xs, s_first + (i + kD) * stride);
    }
  }
};

// A 64-bit value every lane of the wave holds, made a scalar (SGPR) value for the compiler.
__device__ __forceinline__ int64_t mf_uniform(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Half 0 + half 1 of every tile in registers: afterwards lane q' = m + 16 t4 (m < 8, t4 < 2) holds, in element t,
// the wave's partial sum for row 4 t4 + t of the block and activation row m of the activation block.
template <int RB, int MB>
__device__ __forceinline__ void mf_fold_halves(floatx4 (&acc)[RB][MB]) {
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      floatx4 v = acc[rb][b];
      v.x += __shfl_down(v.x, 40);
      v.y += __shfl_down(v.y, 40);
      v.z += __shfl_down(v.z, 40);
      v.w += __shfl_down(v.w, 40);
      acc[rb][b] = v;
    }
}

// LDS image of the folded wave tiles: red[wave][rb][b][q][t], q = m + 8 (row / 4), t = row % 4.
template <int WAVES, int RB, int MB>
struct MfRed {
  float v[WAVES][RB][MB][16][4];
};

template <int WAVES, int RB, int MB>
__device__ __forceinline__ void mf_store_red(MfRed<WAVES, RB, MB>& red, const floatx4 (&acc)[RB][MB], int wave,
                                             int lane) {
  const int q = (lane & 7) + 8 * (lane >> 4);
  if ((lane & 15) < 8 && lane < 32) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        *reinterpret_cast<floatx4*>(&red.v[wave][rb][b][q][0]) = acc[rb][b];
      }
  }
}

// Total of output (row rr of the workgroup's 8 RB rows, activation row m): the folded wave partials in wave order.
template <int WAVES, int RB, int MB>
__device__ __forceinline__ float mf_total(const MfRed<WAVES, RB, MB>& red, int rr, int m) {
  const int rb = rr >> 3, r = rr & 7, b = m >> 3;
  const int q = (m & 7) + 8 * (r >> 2), t = r & 3;
  float tot = red.v[0][rb][b][q][t];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) tot += red.v[w][rb][b][q][t];
  return tot;
}

// Register-budget depth: segments in flight per wave.
template <int KIND, int MB, int RB, bool XMEM>
constexpr int mf_depth() {
  constexpr int slot = 4 * (RB + (XMEM ? MB * MfGeom<KIND>::kParts : 0));
  constexpr int d = 96 / slot;
  return d < 2 ? 2 : d > 8 ? 8 : d;
}

}  // namespace bp
