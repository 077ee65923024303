// Fused multi-step mLSTM recurrence for gfx950 (batch 1): T positions per launch from a read-only start state,
// writing only the cell outputs h_t (and copies of the start n, m).
//
// Per position t of head hd (f and i are gate pre-activations):
//   fl = log(sigmoid(f_t)); m_t = max(fl + m_{t-1}, i_t)
//   fa = io(exp(fl + m_{t-1} - m_t)); ia = io(exp(i_t - m_t)); mv = io(exp(-m_t))      (io = round to io dtype)
//   C_t = fa C_{t-1} + ia k_t v_t^T;  n_t = fa n_{t-1} + ia k_t                          (fp32 state)
//   h_t = (qs . io(C_t)) / (max(|qs . io(n_t)|, mv) + eps),  qs = q_t * qk_scale          (stored as io dtype)
//
// Layout: workgroup (value block b, head hd) owns the columns [b*BV, b*BV + BV) of C for every dq; thread t owns
// the DPT rows dq = t + j * threads of that column block in registers, for the whole launch.
// The recurrence itself is elementwise (C_t depends only on C_{t-1} in the same registers); only the outputs need
// reductions over dq. Those are deferred and batched: G = 64 / BV positions are advanced, their G x BV partial
// dot products are then added across the wave in one transposing butterfly (wave_transpose_reduce<64>) and across
// waves in LDS, so the dependent chain per position is a handful of FMAs and one reduction serves G positions.
// The scalar gate chain (m_t) runs across lanes: lane g computes the activations of position t0 + g.
// Latency: every load of a group is unconditional and issued in the order of use (start state, gates, v, q, k),
// so each wait is an exact count; v reaches the lanes by readlane, the butterflies run in the VALU (permlane swaps
// and DPP), and full groups are compiled without per-position checks.
//
// Reference semantics: byteprof/optim/mlstm_multistep.py:21-30 (_gates), :34-86 (multistep_fw_kernel);
// byteprof/optim/draft_fused.py:27-40 (multistep_fw).

#include "byteprof_amd.h"
#include "common.h"

#include <type_traits>

// Timeline builds (-DBP_TIMELINE, `python -m byteprof_amd.build --timeline`, a separate library): thread 0 of
// every workgroup of the multistep kernel stamps s_memrealtime (100 MHz) at the kernel's stages into
// bp_mlstm_timeline[workgroup][8], which bp_mlstm_timeline_read() copies out: 0 entry, 1 every load of the first
// group landed (an explicit wait for all loads, which a normal build leaves to the first use), 2 the gate chain
// (m_t and the activations) done, 3 the 16 positions' state updates done, 4 the in-wave reductions done, 5 the
// cross-wave sums combined (after the barrier), 6 the outputs stored (after the barrier), 7 the end. Normal builds
// compile none of it.
#ifdef BP_TIMELINE
__device__ unsigned long long bp_mlstm_timeline[1024][8];
extern "C" int bp_mlstm_timeline_read(void* dst, size_t bytes) {
  if (bytes < sizeof(bp_mlstm_timeline)) return BP_E_INVALID_ARG;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(bp_mlstm_timeline), sizeof(bp_mlstm_timeline)) == hipSuccess
             ? BP_OK
             : BP_E_INVALID_ARG;
}
#define BP_TL(k)                                                 \
  do {                                                           \
    if (threadIdx.x == 0) tl_[k] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define BP_TL(k) \
  do {           \
  } while (0)
#endif

namespace bp {
namespace {

template <int IO>
__device__ __forceinline__ float load_io(const void* p, int64_t i) {
  if constexpr (IO == BP_DT_BF16) return bf16_bits_to_float(static_cast<const uint16_t*>(p)[i]);
  else if constexpr (IO == BP_DT_F16) return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  else return static_cast<const float*>(p)[i];
}

template <int IO>
__device__ __forceinline__ float round_io(float f) {
  if constexpr (IO == BP_DT_BF16) return round_to_bf16(f);
  else if constexpr (IO == BP_DT_F16) return round_to_f16(f);
  else return f;
}

template <int IO>
__device__ __forceinline__ void store_io(void* p, int64_t i, float f) {
  if constexpr (IO == BP_DT_BF16) static_cast<uint16_t*>(p)[i] = float_to_bf16_bits(f);
  else if constexpr (IO == BP_DT_F16) static_cast<_Float16*>(p)[i] = static_cast<_Float16>(f);
  else static_cast<float*>(p)[i] = f;
}

// The raw bits of an io_dtype element (loaded without converting, so a batch of loads stays in flight) and their
// value.
template <int IO>
__device__ __forceinline__ uint32_t load_raw(const void* p, int64_t i) {
  if constexpr (IO == BP_DT_F32) return static_cast<const uint32_t*>(p)[i];
  else return static_cast<const uint16_t*>(p)[i];
}

template <int IO>
__device__ __forceinline__ float raw_value(uint32_t r) {
  if constexpr (IO == BP_DT_BF16) return bf16_bits_to_float(r);
  else if constexpr (IO == BP_DT_F16) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r)));
  else return __uint_as_float(r);
}

// log(sigmoid(f)) = -log(1 + exp(-f)), with HIP's fast exp and log (the hardware's exp2 / log2, ~1 ulp); the
// activations use __expf too (the lazy commit the same, so a step and a multistep-then-commit agree bit for bit):
// the gate chain heads every position's dependent work, and the library expf / logf / division were most of it.
__device__ __forceinline__ float log_sigmoid(float f) { return -__logf(1.f + __expf(-f)); }

// One step of the gate chain's scan: compose each lane's max-plus map (A, B) with the one D lanes below it
// (row_shr:D; the group's G <= 16 lanes are in the first row, and lanes below D read the identity (-inf, 0)).
template <int D, int G>
__device__ __forceinline__ void scan_step(float& A, float& B) {
  if constexpr (D < G) {
    const float Ad = __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(-__builtin_huge_valf()), __float_as_int(A), 0x110 + D, 0xF, 0xF,
                                    false));
    const float Bd = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(B), 0x110 + D, 0xF, 0xF, false));
    A = fmaxf(A, B + Ad);
    B = B + Bd;
  }
}

// bf16(lo) | bf16(hi) << 16, both rounded to nearest even (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

__device__ __forceinline__ float load_gate(const void* p, int64_t i, int dt) {
  if (dt == BP_DT_BF16) return bf16_bits_to_float(static_cast<const uint16_t*>(p)[i]);
  if (dt == BP_DT_F16) return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

// A gate element as two raw 16-bit halves: a 4-byte gate is read as its two halves, a 2-byte gate twice, so the
// loads are the same two instructions for every gate dtype (no branch between loads that would force a full wait).
struct GateRaw {
  uint32_t lo, hi;
};

__device__ __forceinline__ GateRaw load_gate_raw(const void* p, int64_t i, int dt) {
  const auto b = as_global(static_cast<const uint16_t*>(p));
  const int64_t e = dt == BP_DT_F32 ? 2 * i : i;
  return {b[e], b[e + (dt == BP_DT_F32 ? 1 : 0)]};
}

__device__ __forceinline__ float gate_value(GateRaw r, int dt) {
  if (dt == BP_DT_F32) return __uint_as_float(r.lo | (r.hi << 16));
  if (dt == BP_DT_BF16) return bf16_bits_to_float(r.lo);
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.lo)));
}

constexpr int kMaxWaves = 4;

template <int IO, int BV, int DPT>
__global__ __launch_bounds__(kMaxWaves * kWave) void mlstm_multistep_kernel(
    const float* __restrict__ c, const float* __restrict__ n, const float* __restrict__ m,
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    const void* __restrict__ ig, const void* __restrict__ fg, void* __restrict__ h, float* __restrict__ nstart,
    float* __restrict__ mstart, float* __restrict__ c_out, float* __restrict__ n_out, float* __restrict__ m_out,
    int T, int DQ, int DV, int64_t str_qk, int64_t str_v, int64_t str_if, int64_t str_h, int gate_dt,
    float qk_scale, float eps) {
  constexpr int G = kWave / BV;  // positions per reduction group
  __shared__ float red_h[kMaxWaves][kWave];
  __shared__ float red_q[kMaxWaves][G];

  const int hd = blockIdx.y;
  const int v0 = blockIdx.x * BV;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int nthreads = blockDim.x;
  const int nwaves = nthreads / kWave;
#ifdef BP_TIMELINE
  unsigned long long tl_[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#endif
  BP_TL(0);

  // This thread's block of the start state, loaded first (the loop keeps a copy of the start n, whose wait then
  // covers only these loads).
  float C[DPT][BV];
  float nn[DPT], n_start[DPT];
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int dq = tid + j * nthreads;
    const float* crow = c + (static_cast<int64_t>(hd) * DQ + dq) * DV + v0;
#pragma unroll
    for (int b = 0; b < BV; ++b) C[j][b] = crow[b];
    nn[j] = n_start[j] = n[static_cast<int64_t>(hd) * DQ + dq];
  }
  float m_prev = m[hd];
  const float m_start = m_prev;

  // Everything a group of G positions reads, as raw bits, issued in the order it is needed: lane g's gate
  // pre-activations of position t0 + g (they head the longest dependent chain), lane l's v element (position
  // t0 + l / BV, column v0 + l % BV), then this thread's q and k rows. Positions past T read the group's last
  // position, unused; every load is unconditional, so the waits for them are exact counts.
  GateRaw fr, ir;
  uint32_t vr;
  uint32_t qv[G][DPT], kv[G][DPT];
  auto issue_group = [&](int t0) {
    const int last = (T - t0 < G ? T - t0 : G) - 1;
    const int64_t goff = static_cast<int64_t>(t0 + (lane < last ? lane : last)) * str_if + hd;
    fr = load_gate_raw(fg, goff, gate_dt);
    ir = load_gate_raw(ig, goff, gate_dt);
    const int vg = lane / BV < last ? lane / BV : last;
    vr = load_raw<IO>(v, static_cast<int64_t>(t0 + vg) * str_v + static_cast<int64_t>(hd) * DV + v0 + lane % BV);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < DPT; ++j) {
        const int64_t qk_off = static_cast<int64_t>(t0 + (g < last ? g : last)) * str_qk +
                               static_cast<int64_t>(hd) * DQ + tid + j * nthreads;
        qv[g][j] = load_raw<IO>(q, qk_off);
        kv[g][j] = load_raw<IO>(k, qk_off);
      }
  };
  __builtin_assume(T >= 1);  // the host handles T = 0 without a launch
  issue_group(0);
#ifdef BP_TIMELINE
  __builtin_amdgcn_s_waitcnt(0);
  BP_TL(1);
#endif

  for (int t0 = 0; t0 < T; t0 += G) {
    const int gcount = T - t0 < G ? T - t0 : G;

    // The gate chain and the state advance over the group's positions; a full group (every group but a last,
    // partial one) is compiled without the per-position checks.
    float hp[G * BV];
    float qp[G];
    float mv_l;
    auto advance = [&](auto full) {
      constexpr bool FULL = decltype(full)::value;
      // Gate activations: lane g < gcount handles position t0 + g; the max-plus chain of m runs through the lanes.
      const float fv = gate_value(fr, gate_dt);
      const float iv = gate_value(ir, gate_dt);
      const float fl = log_sigmoid(fv);
      // m over the group as an inclusive scan across lanes 0 .. G - 1 of the max-plus maps x -> max(i_t, fl_t + x):
      // a map is (A, B) = x -> max(A, B + x); (A2, B2) after (A1, B1) is (max(A2, B2 + A1), B2 + B1); lanes past
      // gcount hold the identity (-inf, 0). log2(G) steps of row shifts instead of G dependent broadcasts.
      const bool pos = FULL || lane < gcount;
      float A = pos ? iv : -__builtin_huge_valf();
      float B = pos ? fl : 0.f;
      scan_step<1, G>(A, B);
      scan_step<2, G>(A, B);
      scan_step<4, G>(A, B);
      scan_step<8, G>(A, B);
      const float m_new_l = fmaxf(A, B + m_prev);  // m of position t0 + lane
      const float m_old_l = __int_as_float(  // m of the position before
          __builtin_amdgcn_update_dpp(__float_as_int(m_prev), __float_as_int(m_new_l), 0x111, 0xF, 0xF, false));
      m_prev = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m_new_l), gcount - 1));
      const float fa_l = round_io<IO>(__expf(fl + m_old_l - m_new_l));
      const float ia_l = round_io<IO>(__expf(iv - m_new_l));
      mv_l = round_io<IO>(__expf(-m_new_l));
      const float v_l = raw_value<IO>(vr);
      BP_TL(2);

      // Advance the state over the group's positions, keeping the per-thread partial dot products.
#pragma unroll
      for (int g = 0; g < G; ++g) {
        qp[g] = 0.f;
#pragma unroll
        for (int b = 0; b < BV; ++b) hp[g * BV + b] = 0.f;
        if (FULL || g < gcount) {
          const float fa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fa_l), g));
          const float ia = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ia_l), g));
          float vv[BV];
#pragma unroll
          for (int b = 0; b < BV; ++b)
            vv[b] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v_l), g * BV + b));
#pragma unroll
          for (int j = 0; j < DPT; ++j) {
            const float kk = raw_value<IO>(kv[g][j]);
            const float ik = ia * kk;
            if constexpr (IO == BP_DT_BF16) {
              // bf16 io: the rounded state enters the dot products as packed bf16 pairs (one conversion per two
              // columns) against q unscaled, (q, 0) for the even column and (0, q) for the odd one (v_dot2_f32_bf16:
              // exact products, the same sums up to the order of rounding); qk_scale is applied to the sums
              const uint32_t qlo = qv[g][j], qhi = qv[g][j] << 16;
#pragma unroll
              for (int b = 0; b < BV; b += 2) {
                C[j][b] = fmaf(ik, vv[b], fa * C[j][b]);
                C[j][b + 1] = fmaf(ik, vv[b + 1], fa * C[j][b + 1]);
                const uint32_t pk = pack_bf16x2(C[j][b], C[j][b + 1]);
                hp[g * BV + b] = dot2_bf16(pk, qlo, hp[g * BV + b]);
                hp[g * BV + b + 1] = dot2_bf16(pk, qhi, hp[g * BV + b + 1]);
              }
              nn[j] = fmaf(fa, nn[j], ik);
              qp[g] = dot2_bf16(pack_bf16x2(nn[j], 0.f), qlo, qp[g]);
            } else {
              const float qs = raw_value<IO>(qv[g][j]) * qk_scale;
#pragma unroll
              for (int b = 0; b < BV; ++b) {
                C[j][b] = fmaf(ik, vv[b], fa * C[j][b]);
                hp[g * BV + b] = fmaf(qs, round_io<IO>(C[j][b]), hp[g * BV + b]);
              }
              nn[j] = fmaf(fa, nn[j], ik);
              qp[g] = fmaf(qs, round_io<IO>(nn[j]), qp[g]);
            }
          }
        }
        // one position's broadcasts (scalar registers) at a time: hoisted for all positions they spill
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (gcount == G) advance(std::true_type{});
    else advance(std::false_type{});
    BP_TL(3);

    if (t0 + G < T) issue_group(t0 + G);  // the next group's loads, in flight during the reductions

    wave_transpose_reduce<G * BV>(hp, lane);  // lane l: wave total of index l = g * BV + b
    wave_transpose_reduce<G>(qp, lane);       // lane l: wave total of position l / (64 / G)
    BP_TL(4);
    red_h[wave][lane] = hp[0];
    if ((lane & (kWave / G - 1)) == 0) red_q[wave][lane / (kWave / G)] = qp[0];
    __syncthreads();
    BP_TL(5);
    if (wave == 0) {
      const int g = lane / BV;
      float hs = red_h[0][lane];
      float qn = red_q[0][g];
      for (int w = 1; w < nwaves; ++w) {
        hs += red_h[w][lane];
        qn += red_q[w][g];
      }
      const float mv = __shfl(mv_l, g);
      if constexpr (IO == BP_DT_BF16) {
        hs *= qk_scale;
        qn *= qk_scale;
      }
      if (g < gcount) {
        const float out = hs / (fmaxf(fabsf(qn), mv) + eps);
        store_io<IO>(h, static_cast<int64_t>(t0 + g) * str_h + static_cast<int64_t>(hd) * DV + v0 + (lane % BV),
                     out);
      }
    }
    __syncthreads();
    BP_TL(6);
  }
  // copies of the start n and m (stored last, so no wait for their loads delays the gate chain)
  if (blockIdx.x == 0 && nstart != nullptr) {
#pragma unroll
    for (int j = 0; j < DPT; ++j) nstart[static_cast<int64_t>(hd) * DQ + tid + j * nthreads] = n_start[j];
    if (tid == 0 && mstart != nullptr) mstart[hd] = m_start;
  }
  // the state after the last position, into the caller's buffers (a step writing its new state)
  if (c_out != nullptr) {
#pragma unroll
    for (int j = 0; j < DPT; ++j) {
      const int dq = tid + j * nthreads;
      float* crow = c_out + (static_cast<int64_t>(hd) * DQ + dq) * DV + v0;
#pragma unroll
      for (int b = 0; b < BV; ++b) crow[b] = C[j][b];
      if (blockIdx.x == 0) n_out[static_cast<int64_t>(hd) * DQ + dq] = nn[j];
    }
    if (blockIdx.x == 0 && tid == 0) m_out[hd] = m_prev;
  }
  BP_TL(7);
#ifdef BP_TIMELINE
  const int wg = blockIdx.y * gridDim.x + blockIdx.x;
  if (threadIdx.x == 0 && wg < 1024)
    for (int e = 0; e < 8; ++e) bp_mlstm_timeline[wg][e] = tl_[e];
#endif
}

// Lazy commit of a verify round: the state after positions 0 .. L (L read from device memory, so a captured graph
// serves every accepted length), recomputed from the start state with the round's saved k, v and gates: C is the
// start C on entry (multistep left it untouched) and is updated in place; n and m start from nstart / mstart (the
// copies multistep made) and are written to n and m. Positions are clamped to the T that k, v, i, f hold. The
// recurrence is elementwise, so a thread carries its DPT x BV block of C (and its n rows) through all positions with
// no reduction; the gate chain is computed by every thread the same way as in mlstm_multistep_kernel.
// Reference semantics: byteprof/optim/mlstm_multistep.py:89-134 (lazy_commit_kernel), draft_fused.py:43-56.
template <int IO, int BV, int DPT>
__global__ __launch_bounds__(kMaxWaves * kWave) void mlstm_lazy_commit_kernel(
    float* __restrict__ c, float* __restrict__ n, float* __restrict__ m, const float* __restrict__ nstart,
    const float* __restrict__ mstart, const void* __restrict__ k, const void* __restrict__ v,
    const void* __restrict__ ig, const void* __restrict__ fg, const int64_t* __restrict__ length, int T, int DQ,
    int DV, int64_t str_qk, int64_t str_v, int64_t str_if, int gate_dt) {
  const int hd = blockIdx.y;
  const int v0 = blockIdx.x * BV;
  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;
  const int64_t L = *length;
  const int npos = L < 0 ? 0 : (L + 1 > T ? T : static_cast<int>(L + 1));

  float C[DPT][BV];
  float nn[DPT];
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int dq = tid + j * nthreads;
    const float* crow = c + (static_cast<int64_t>(hd) * DQ + dq) * DV + v0;
#pragma unroll
    for (int b = 0; b < BV; ++b) C[j][b] = crow[b];
    nn[j] = nstart[static_cast<int64_t>(hd) * DQ + dq];
  }
  float m_prev = mstart[hd];
  for (int t = 0; t < npos; ++t) {
    const int64_t off = static_cast<int64_t>(t) * str_if + hd;
    const float fv = load_gate(fg, off, gate_dt);
    const float iv = load_gate(ig, off, gate_dt);
    const float fl = log_sigmoid(fv);
    const float mn = fmaxf(fl + m_prev, iv);
    const float fa = round_io<IO>(__expf(fl + m_prev - mn));
    const float ia = round_io<IO>(__expf(iv - mn));
    m_prev = mn;
    float vv[BV];
#pragma unroll
    for (int b = 0; b < BV; ++b) vv[b] = load_io<IO>(v, static_cast<int64_t>(t) * str_v + static_cast<int64_t>(hd) * DV + v0 + b);
#pragma unroll
    for (int j = 0; j < DPT; ++j) {
      const int dq = tid + j * nthreads;
      const float ik = ia * load_io<IO>(k, static_cast<int64_t>(t) * str_qk + static_cast<int64_t>(hd) * DQ + dq);
#pragma unroll
      for (int b = 0; b < BV; ++b) C[j][b] = fmaf(ik, vv[b], fa * C[j][b]);
      nn[j] = fmaf(fa, nn[j], ik);
    }
  }
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int dq = tid + j * nthreads;
    float* crow = c + (static_cast<int64_t>(hd) * DQ + dq) * DV + v0;
#pragma unroll
    for (int b = 0; b < BV; ++b) crow[b] = C[j][b];
    if (blockIdx.x == 0) n[static_cast<int64_t>(hd) * DQ + dq] = nn[j];
  }
  if (blockIdx.x == 0 && tid == 0) m[hd] = m_prev;
}

using CommitFn = void (*)(float*, float*, float*, const float*, const float*, const void*, const void*, const void*,
                          const void*, const int64_t*, int, int, int, int64_t, int64_t, int64_t, int);

template <int IO, int BV>
CommitFn commit_dpt(int dpt) {
  return dpt == 1 ? &mlstm_lazy_commit_kernel<IO, BV, 1> : &mlstm_lazy_commit_kernel<IO, BV, 2>;
}

template <int IO>
CommitFn commit_bv(int bv, int dpt) {
  switch (bv) {
    case 4: return commit_dpt<IO, 4>(dpt);
    case 8: return commit_dpt<IO, 8>(dpt);
    case 16: return commit_dpt<IO, 16>(dpt);
    default: return nullptr;
  }
}

CommitFn pick_commit(int io, int bv, int dpt) {
  switch (io) {
    case BP_DT_BF16: return commit_bv<BP_DT_BF16>(bv, dpt);
    case BP_DT_F16: return commit_bv<BP_DT_F16>(bv, dpt);
    case BP_DT_F32: return commit_bv<BP_DT_F32>(bv, dpt);
    default: return nullptr;
  }
}

using MlstmFn = void (*)(const float*, const float*, const float*, const void*, const void*, const void*,
                         const void*, const void*, void*, float*, float*, float*, float*, float*, int, int, int,
                         int64_t, int64_t, int64_t, int64_t, int, float, float);

template <int IO, int BV>
MlstmFn pick_dpt(int dpt) {
  return dpt == 1 ? &mlstm_multistep_kernel<IO, BV, 1> : &mlstm_multistep_kernel<IO, BV, 2>;
}

template <int IO>
MlstmFn pick_bv(int bv, int dpt) {
  switch (bv) {
    case 4: return pick_dpt<IO, 4>(dpt);
    case 8: return pick_dpt<IO, 8>(dpt);
    case 16: return pick_dpt<IO, 16>(dpt);
    default: return nullptr;
  }
}

MlstmFn pick(int io, int bv, int dpt) {
  switch (io) {
    case BP_DT_BF16: return pick_bv<BP_DT_BF16>(bv, dpt);
    case BP_DT_F16: return pick_bv<BP_DT_F16>(bv, dpt);
    case BP_DT_F32: return pick_bv<BP_DT_F32>(bv, dpt);
    default: return nullptr;
  }
}

}  // namespace
}  // namespace bp

namespace bp {
namespace {

// Workgroups of DQ / dpt threads (dpt = 1 up to 256, else 2): whole waves only, so DQ a multiple of 64 up to 256,
// or 384 / 512.
int mlstm_dpt(int DQ) {
  if (DQ <= 0 || DQ % kWave != 0 || DQ > 2 * kMaxWaves * kWave) return 0;
  const int dpt = DQ <= kMaxWaves * kWave ? 1 : 2;
  return (DQ / dpt) % kWave == 0 ? dpt : 0;
}

int mlstm_launch(const void* c, const void* n, const void* m, const void* q, const void* k, const void* v,
                 const void* i, const void* f, void* h, void* nstart, void* mstart, void* c_out, void* n_out,
                 void* m_out, int T, int NH, int DQ, int DV, int64_t str_t_qk, int64_t str_t_v, int64_t str_t_if,
                 int64_t str_t_h, int io_dtype, int gate_dtype, float qk_scale, float eps, int bv, void* stream) {
  if (T < 0 || NH < 0 || DQ <= 0 || DV <= 0) return BP_E_INVALID_ARG;
  if (NH == 0) return BP_OK;
  if (c == nullptr || n == nullptr || m == nullptr) return BP_E_INVALID_ARG;
  if (T > 0 && (q == nullptr || k == nullptr || v == nullptr || i == nullptr || f == nullptr || h == nullptr))
    return BP_E_INVALID_ARG;
  const int dpt = mlstm_dpt(DQ);
  if (dpt == 0) return BP_E_UNSUPPORTED;
  if (gate_dtype < BP_DT_BF16 || gate_dtype > BP_DT_F32) return BP_E_UNSUPPORTED;
  if (bv != 4 && bv != 8 && bv != 16) return BP_E_UNSUPPORTED;
  if (DV % bv != 0) return BP_E_UNSUPPORTED;
  MlstmFn fn = pick(io_dtype, bv, dpt);
  if (fn == nullptr) return BP_E_UNSUPPORTED;
  const auto st = static_cast<hipStream_t>(stream);
  if (T == 0) {  // no positions: the start-state copies are the whole result
    if (nstart == nullptr) return BP_OK;
    hipError_t e = hipMemcpyAsync(nstart, n, sizeof(float) * NH * DQ, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(mstart, m, sizeof(float) * NH, hipMemcpyDeviceToDevice, st);
    return e == hipSuccess ? BP_OK : static_cast<int>(e);
  }
  dim3 grid(static_cast<unsigned>(DV / bv), static_cast<unsigned>(NH));
  fn<<<grid, DQ / dpt, 0, st>>>(
      static_cast<const float*>(c), static_cast<const float*>(n), static_cast<const float*>(m), q, k, v, i, f, h,
      static_cast<float*>(nstart), static_cast<float*>(mstart), static_cast<float*>(c_out),
      static_cast<float*>(n_out), static_cast<float*>(m_out), T, DQ, DV, str_t_qk, str_t_v, str_t_if, str_t_h,
      gate_dtype, qk_scale, eps);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}

}  // namespace
}  // namespace bp

extern "C" int bp_mlstm_step(const void* c, const void* n, const void* m, const void* q, const void* k, const void* v,
                             const void* i, const void* f, void* h, void* c_new, void* n_new, void* m_new, int NH,
                             int DQ, int DV, int io_dtype, int gate_dtype, float qk_scale, float eps, int bv,
                             void* stream) {
  if (c_new == nullptr || n_new == nullptr || m_new == nullptr) return BP_E_INVALID_ARG;
  return bp::mlstm_launch(c, n, m, q, k, v, i, f, h, nullptr, nullptr, c_new, n_new, m_new, 1, NH, DQ, DV,
                          static_cast<int64_t>(NH) * DQ, static_cast<int64_t>(NH) * DV, NH,
                          static_cast<int64_t>(NH) * DV, io_dtype, gate_dtype, qk_scale, eps, bv, stream);
}

extern "C" int bp_mlstm_multistep(const void* c, const void* n, const void* m, const void* q, const void* k,
                                  const void* v, const void* i, const void* f, void* h, void* nstart, void* mstart,
                                  int T, int NH, int DQ, int DV, int64_t str_t_qk, int64_t str_t_v,
                                  int64_t str_t_if, int64_t str_t_h, int io_dtype, int gate_dtype, float qk_scale,
                                  float eps, int bv, void* stream) {
  if (nstart == nullptr || mstart == nullptr) return BP_E_INVALID_ARG;
  return bp::mlstm_launch(c, n, m, q, k, v, i, f, h, nstart, mstart, nullptr, nullptr, nullptr, T, NH, DQ, DV,
                          str_t_qk, str_t_v, str_t_if, str_t_h, io_dtype, gate_dtype, qk_scale, eps, bv, stream);
}

extern "C" int bp_mlstm_lazy_commit(void* c, void* n, void* m, const void* nstart, const void* mstart, const void* k,
                                    const void* v, const void* i, const void* f, const void* length, int T, int NH,
                                    int DQ, int DV, int64_t str_t_qk, int64_t str_t_v, int64_t str_t_if,
                                    int io_dtype, int gate_dtype, int bv, void* stream) {
  if (T < 0 || NH < 0 || DQ <= 0 || DV <= 0) return BP_E_INVALID_ARG;
  if (NH == 0) return BP_OK;
  if (c == nullptr || n == nullptr || m == nullptr || nstart == nullptr || mstart == nullptr || length == nullptr)
    return BP_E_INVALID_ARG;
  if (T > 0 && (k == nullptr || v == nullptr || i == nullptr || f == nullptr)) return BP_E_INVALID_ARG;
  const int dpt = bp::mlstm_dpt(DQ);
  if (dpt == 0) return BP_E_UNSUPPORTED;
  if (gate_dtype < BP_DT_BF16 || gate_dtype > BP_DT_F32) return BP_E_UNSUPPORTED;
  if (bv != 4 && bv != 8 && bv != 16) return BP_E_UNSUPPORTED;
  if (DV % bv != 0) return BP_E_UNSUPPORTED;
  bp::CommitFn fn = bp::pick_commit(io_dtype, bv, dpt);
  if (fn == nullptr) return BP_E_UNSUPPORTED;
  dim3 grid(static_cast<unsigned>(DV / bv), static_cast<unsigned>(NH));
  fn<<<grid, DQ / dpt, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<float*>(c), static_cast<float*>(n), static_cast<float*>(m), static_cast<const float*>(nstart),
      static_cast<const float*>(mstart), k, v, i, f, static_cast<const int64_t*>(length), T, DQ, DV, str_t_qk,
      str_t_v, str_t_if, gate_dtype);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}
