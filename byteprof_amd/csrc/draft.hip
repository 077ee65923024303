// Small device-side steps of a drafting round (batch 1), so that a captured graph needs no host read: the accepted
// length of a verify pass and the commit of the matching state from a per-position history.
//
// Reference semantics: byteprof/optim/mlstm_multistep.py:136-146 (accept_kernel), byteprof/optim/draft_kernels.py
// (commit_kernel) via draft_core.commit_state (draft_core.py:92-111).

#include "byteprof_amd.h"
#include "common.h"

namespace bp {
namespace {

// L = the number of leading drafts ids[1 + j] equal to tok[j] (j < S - 1), by one wave: 64 comparisons per
// ballot, the first mismatch ends the count. Wave-uniform result.
__device__ int64_t accepted_length(const int64_t* __restrict__ ids, const int64_t* __restrict__ tok, int S) {
  const int lane = threadIdx.x;
  int64_t accepted = 0;
  bool open = true;  // wave-uniform: no mismatch seen yet
  for (int j0 = 0; j0 < S - 1 && open; j0 += kWave) {
    const int j = j0 + lane;
    const bool miss = j < S - 1 && ids[1 + j] != tok[j];
    const uint64_t mask = __ballot(miss);
    const int in_range = min(kWave, S - 1 - j0);
    if (mask != 0) {
      accepted += __builtin_ctzll(mask);
      open = false;
    } else {
      accepted += in_range;
    }
  }
  return accepted;
}

// out[:S] <- tok[:S]; out[SMAX] <- L.
__global__ __launch_bounds__(kWave) void draft_accept_kernel(const int64_t* __restrict__ ids,
                                                             const int64_t* __restrict__ tok,
                                                             int64_t* __restrict__ out, int S, int SMAX) {
  const int64_t accepted = accepted_length(ids, tok, S);
  for (int j = threadIdx.x; j < S; j += kWave) out[j] = tok[j];
  if (threadIdx.x == 0) out[SMAX] = accepted;
}

// As draft_accept_kernel, then ids[0] <- tok[L] and *pos += L + 1 (the next verify round's inputs). The drafts
// ids[1 ..] are read before ids[0] is written (the comparisons never read ids[0]).
__global__ __launch_bounds__(kWave) void draft_verify_next_kernel(int64_t* __restrict__ ids,
                                                                  const int64_t* __restrict__ tok,
                                                                  int64_t* __restrict__ out, int64_t* __restrict__ pos,
                                                                  int S, int SMAX) {
  const int64_t accepted = accepted_length(ids, tok, S);
  for (int j = threadIdx.x; j < S; j += kWave) out[j] = tok[j];
  if (threadIdx.x == 0) {
    out[SMAX] = accepted;
    ids[0] = tok[accepted];
    *pos += accepted + 1;
  }
}

// cur <- hist[slot] for one layer's state (c, n, m), slot = *length read on the device (clamped to the history).
__global__ void draft_commit_kernel(const float* __restrict__ c_hist, float* __restrict__ c_cur,
                                    const float* __restrict__ n_hist, float* __restrict__ n_cur,
                                    const float* __restrict__ m_hist, float* __restrict__ m_cur,
                                    const int64_t* __restrict__ length, int64_t slots, int64_t c_n, int64_t n_n,
                                    int64_t m_n) {
  int64_t slot = *length;
  slot = slot < 0 ? 0 : (slot >= slots ? slots - 1 : slot);
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < c_n;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    c_cur[idx] = c_hist[slot * c_n + idx];
    if (idx < n_n) n_cur[idx] = n_hist[slot * n_n + idx];
    if (idx < m_n) m_cur[idx] = m_hist[slot * m_n + idx];
  }
}

}  // namespace
}  // namespace bp

extern "C" {

int bp_draft_verify_next(void* ids, const void* tok, void* out, int64_t* pos, int S, int SMAX, void* stream) {
  if (ids == nullptr || tok == nullptr || out == nullptr || pos == nullptr || S < 1 || SMAX < S)
    return BP_E_INVALID_ARG;
  bp::draft_verify_next_kernel<<<1, bp::kWave, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<int64_t*>(ids), static_cast<const int64_t*>(tok), static_cast<int64_t*>(out), pos, S, SMAX);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}

int bp_draft_accept(const void* ids, const void* tok, void* out, int S, int SMAX, void* stream) {
  if (ids == nullptr || tok == nullptr || out == nullptr || S < 0 || SMAX < S) return BP_E_INVALID_ARG;
  bp::draft_accept_kernel<<<1, bp::kWave, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const int64_t*>(ids), static_cast<const int64_t*>(tok), static_cast<int64_t*>(out), S, SMAX);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}

int bp_draft_commit(const void* c_hist, void* c_cur, const void* n_hist, void* n_cur, const void* m_hist,
                    void* m_cur, const void* length, int64_t slots, int64_t c_n, int64_t n_n, int64_t m_n,
                    void* stream) {
  if (c_hist == nullptr || c_cur == nullptr || n_hist == nullptr || n_cur == nullptr || m_hist == nullptr ||
      m_cur == nullptr || length == nullptr || slots <= 0 || c_n < 0 || n_n < 0 || m_n < 0 || n_n > c_n ||
      m_n > c_n)
    return BP_E_INVALID_ARG;
  if (c_n == 0) return BP_OK;
  const int64_t blocks64 = (c_n + 255) / 256;
  const unsigned blocks = static_cast<unsigned>(blocks64 < 4096 ? blocks64 : 4096);
  bp::draft_commit_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const float*>(c_hist), static_cast<float*>(c_cur), static_cast<const float*>(n_hist),
      static_cast<float*>(n_cur), static_cast<const float*>(m_hist), static_cast<float*>(m_cur),
      static_cast<const int64_t*>(length), slots, c_n, n_n, m_n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}

}  // extern "C"
