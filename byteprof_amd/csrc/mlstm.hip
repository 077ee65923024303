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
//
// Reference semantics: byteprof/optim/mlstm_multistep.py:21-30 (_gates), :34-86 (multistep_fw_kernel);
// byteprof/optim/draft_fused.py:27-40 (multistep_fw).

#include "byteprof_amd.h"
#include "common.h"

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

__device__ __forceinline__ float load_gate(const void* p, int64_t i, int dt) {
  if (dt == BP_DT_BF16) return bf16_bits_to_float(static_cast<const uint16_t*>(p)[i]);
  if (dt == BP_DT_F16) return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

constexpr int kMaxWaves = 4;

template <int IO, int BV, int DPT>
__global__ __launch_bounds__(kMaxWaves * kWave) void mlstm_multistep_kernel(
    const float* __restrict__ c, const float* __restrict__ n, const float* __restrict__ m,
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    const void* __restrict__ ig, const void* __restrict__ fg, void* __restrict__ h, float* __restrict__ nstart,
    float* __restrict__ mstart, int T, int DQ, int DV, int64_t str_qk, int64_t str_v, int64_t str_if,
    int64_t str_h, int gate_dt, float qk_scale, float eps) {
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

  float C[DPT][BV];
  float nn[DPT];
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int dq = tid + j * nthreads;
    const float* crow = c + (static_cast<int64_t>(hd) * DQ + dq) * DV + v0;
#pragma unroll
    for (int b = 0; b < BV; ++b) C[j][b] = crow[b];
    nn[j] = n[static_cast<int64_t>(hd) * DQ + dq];
    if (blockIdx.x == 0) nstart[static_cast<int64_t>(hd) * DQ + dq] = nn[j];
  }
  float m_prev = m[hd];
  if (blockIdx.x == 0 && tid == 0) mstart[hd] = m_prev;

  for (int t0 = 0; t0 < T; t0 += G) {
    const int gcount = T - t0 < G ? T - t0 : G;

    // Gate activations: lane g < gcount handles position t0 + g; the max-plus chain of m runs through the lanes.
    float fl = 0.f, iv = 0.f;
    if (lane < gcount) {
      const int64_t off = static_cast<int64_t>(t0 + lane) * str_if + hd;
      const float fv = load_gate(fg, off, gate_dt);
      iv = load_gate(ig, off, gate_dt);
      fl = logf(1.f / (1.f + expf(-fv)));
    }
    float m_old_l = 0.f, m_new_l = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (g < gcount) {
        const float fg_g = __shfl(fl, g);
        const float ig_g = __shfl(iv, g);
        const float mn = fmaxf(fg_g + m_prev, ig_g);
        if (lane == g) {
          m_old_l = m_prev;
          m_new_l = mn;
        }
        m_prev = mn;
      }
    }
    const float fa_l = round_io<IO>(expf(fl + m_old_l - m_new_l));
    const float ia_l = round_io<IO>(expf(iv - m_new_l));
    const float mv_l = round_io<IO>(expf(-m_new_l));

    // Advance the state over the group's positions, keeping the per-thread partial dot products.
    float hp[G * BV];
    float qp[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      qp[g] = 0.f;
#pragma unroll
      for (int b = 0; b < BV; ++b) hp[g * BV + b] = 0.f;
      if (g < gcount) {
        const int t = t0 + g;
        const float fa = __shfl(fa_l, g);
        const float ia = __shfl(ia_l, g);
        float vv[BV];
#pragma unroll
        for (int b = 0; b < BV; ++b) vv[b] = load_io<IO>(v, static_cast<int64_t>(t) * str_v + static_cast<int64_t>(hd) * DV + v0 + b);
#pragma unroll
        for (int j = 0; j < DPT; ++j) {
          const int dq = tid + j * nthreads;
          const int64_t qk_off = static_cast<int64_t>(t) * str_qk + static_cast<int64_t>(hd) * DQ + dq;
          const float kk = load_io<IO>(k, qk_off);
          const float qs = load_io<IO>(q, qk_off) * qk_scale;
          const float ik = ia * kk;
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

    wave_transpose_reduce<G * BV>(hp, lane);  // lane l: wave total of index l = g * BV + b
    wave_transpose_reduce<G>(qp, lane);       // lane l: wave total of position l / (64 / G)
    red_h[wave][lane] = hp[0];
    if ((lane & (kWave / G - 1)) == 0) red_q[wave][lane / (kWave / G)] = qp[0];
    __syncthreads();
    if (wave == 0) {
      const int g = lane / BV;
      float hs = red_h[0][lane];
      float qn = red_q[0][g];
      for (int w = 1; w < nwaves; ++w) {
        hs += red_h[w][lane];
        qn += red_q[w][g];
      }
      const float mv = __shfl(mv_l, g);
      if (g < gcount) {
        const float out = hs / (fmaxf(fabsf(qn), mv) + eps);
        store_io<IO>(h, static_cast<int64_t>(t0 + g) * str_h + static_cast<int64_t>(hd) * DV + v0 + (lane % BV),
                     out);
      }
    }
    __syncthreads();
  }
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
    const float fl = logf(1.f / (1.f + expf(-fv)));
    const float mn = fmaxf(fl + m_prev, iv);
    const float fa = round_io<IO>(expf(fl + m_prev - mn));
    const float ia = round_io<IO>(expf(iv - mn));
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
                         const void*, const void*, void*, float*, float*, int, int, int, int64_t, int64_t, int64_t,
                         int64_t, int, float, float);

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

extern "C" int bp_mlstm_multistep(const void* c, const void* n, const void* m, const void* q, const void* k,
                                  const void* v, const void* i, const void* f, void* h, void* nstart, void* mstart,
                                  int T, int NH, int DQ, int DV, int64_t str_t_qk, int64_t str_t_v,
                                  int64_t str_t_if, int64_t str_t_h, int io_dtype, int gate_dtype, float qk_scale,
                                  float eps, int bv, void* stream) {
  if (T < 0 || NH < 0 || DQ <= 0 || DV <= 0) return BP_E_INVALID_ARG;
  if (NH == 0) return BP_OK;
  if (c == nullptr || n == nullptr || m == nullptr || nstart == nullptr || mstart == nullptr) return BP_E_INVALID_ARG;
  if (T > 0 && (q == nullptr || k == nullptr || v == nullptr || i == nullptr || f == nullptr || h == nullptr))
    return BP_E_INVALID_ARG;
  if (DQ % bp::kWave != 0 || DQ > 2 * bp::kMaxWaves * bp::kWave) return BP_E_UNSUPPORTED;
  if (gate_dtype < BP_DT_BF16 || gate_dtype > BP_DT_F32) return BP_E_UNSUPPORTED;
  if (bv != 4 && bv != 8 && bv != 16) return BP_E_UNSUPPORTED;
  if (DV % bv != 0) return BP_E_UNSUPPORTED;
  const int dpt = DQ <= bp::kMaxWaves * bp::kWave ? 1 : 2;
  bp::MlstmFn fn = bp::pick(io_dtype, bv, dpt);
  if (fn == nullptr) return BP_E_UNSUPPORTED;
  dim3 grid(static_cast<unsigned>(DV / bv), static_cast<unsigned>(NH));
  fn<<<grid, DQ / dpt, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const float*>(c), static_cast<const float*>(n), static_cast<const float*>(m), q, k, v, i, f, h,
      static_cast<float*>(nstart), static_cast<float*>(mstart), T, DQ, DV, str_t_qk, str_t_v, str_t_if, str_t_h,
      gate_dtype, qk_scale, eps);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
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
  if (DQ % bp::kWave != 0 || DQ > 2 * bp::kMaxWaves * bp::kWave) return BP_E_UNSUPPORTED;
  if (gate_dtype < BP_DT_BF16 || gate_dtype > BP_DT_F32) return BP_E_UNSUPPORTED;
  if (bv != 4 && bv != 8 && bv != 16) return BP_E_UNSUPPORTED;
  if (DV % bv != 0) return BP_E_UNSUPPORTED;
  const int dpt = DQ <= bp::kMaxWaves * bp::kWave ? 1 : 2;
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
