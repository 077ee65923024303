// The decode-step linear set in one launch of the skinny matrix-core kernel (skinny_mf.h): a grid whose workgroups
// are ordered by stage, each workgroup owning 8 rb rows of one linear ("item"), rb chosen per item so that the
// workgroup's whole weight tile is in flight before it needs its input (16 segments per wave). Two modes:
//   - independent (the reference's set benchmark, tools/skinny_bench.py:45-71): every item reads its own input
//     vector; no workgroup waits for another;
//   - dependent (a decode step's chain): an item reads a slice of an earlier stage's output, optionally renormalised
//     to unit RMS. Its workgroups issue their first weight loads, then wait for that output, so the weights stream
//     across stage boundaries while the input is still being computed.
//
// Hand-off between workgroups (dependent mode): a one-thread kernel ahead of the grid advances the launch
// generation g (so no workgroup of the grid ever sees it change). Every output is also stored as a 32-bit word
// [tag : bf16 value] with an agent-scope (device-coherent) store, the tag being (g mod 2^15) + 1, so a word is either
// seen whole and current or recognised as stale -- no fences, and nothing is cleared between launches. A producer
// workgroup issues its stores, then adds 1 to its stage's counter, which therefore only grows: the stage has
// reported in launch g once counter - (g - 1) x (its workgroups) reaches its workgroup count (unsigned arithmetic,
// exact across wrap-around). A consumer polls that counter (a hint that keeps polling off the input words), then
// reads its input words and re-reads any stale one. Every wait is bounded; a wait that gives up sets the error word
// and the launch still finishes.
//
// Deadlock freedom: the hardware dispatches the workgroups of a grid in index order (per XCD), and a workgroup
// only waits for items of lower index; so whenever a stage is incomplete, all of its workgroups have been placed,
// and none of them waits for a later one.
//
// Every output equals bp_skinny_mf's at M = 1 with the same waves and split 1, bit for bit: the same segments per
// wave, the same MFMA chain, the same reductions (the rows per workgroup and the loads in flight do not change a
// row's arithmetic; the activation operand is read from LDS here, from the same values).
//
// Reference semantics: byteprof/optim/skinny.py:36-90 (one-row arithmetic), the set of tools/skinny_bench.py:45-71
// (independent) and the decode step of byteprof/optim/olmo.py:122-219 (dependent: each stage waits for the
// output it needs).

#include <algorithm>

#include "byteprof_amd.h"
#include "skinny_mf.h"

namespace bp {
namespace {

constexpr int kChainKMax = 8192;        // input elements per item (LDS: 16 KiB)
constexpr int kHdrGen = 0;              // scratch words: launch generation
constexpr int kHdrError = 2;            // set by a wait that gave up
constexpr int kHdrCounters = 64;        // first per-stage completion counter
constexpr long kSpinCounter = 1L << 22; // counter polls before giving up
constexpr long kSpinWord = 1L << 16;    // polls of one stale input word before giving up
constexpr int kGatherLoads = 4;         // independent 64-bit input loads in flight per thread (one batch)
constexpr uint32_t kSlackDiv = 8;       // consumers read their words once all but 1/8 of the producers reported

// Device-coherent (agent-scope) accesses, through global-memory views of the pointers.
__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent64(const uint64_t* p) {
  return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(as_global_mut(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The item a workgroup belongs to: lut[b / 256] is the item holding workgroup 256 (b / 256), then a forward walk.
__device__ __forceinline__ int chain_item(const BpChainItem* __restrict__ items, const int32_t* __restrict__ lut,
                                          int n_items, int b) {
  int i = lut[b >> 8];
  while (i + 1 < n_items && items[i + 1].first_wg <= b) ++i;
  return i;
}

// Weight slots in flight per wave: a workgroup of 8 rb rows holds 16 / rb segments per row block, so a tile of
// 8 rb rows x K is in flight whole before the input wait whenever K / (segment x waves) <= 16 / rb.
constexpr int kChainSlots = 16;

// The rows a workgroup owns, in 8-row blocks, for an item of K elements: the most rows whose whole tile fits the
// slots (1, 2 or 4 blocks), or the requested count.
__host__ __device__ constexpr int chain_rb(int64_t nseg_per_wave, int rb_req) {
  return rb_req > 0 ? rb_req : nseg_per_wave <= 4 ? 4 : nseg_per_wave <= 8 ? 2 : 1;
}

struct ChainShared {
  uint16_t xs[kChainKMax];
  float red[8 * 4 * 16 * 4];  // MfRed<waves <= 8, rb <= 4, 1>
  float ss[8];
  int wait_ok;
};

template <int KIND, int RB, int WAVES>
__device__ __forceinline__ void chain_body(const BpChainItem& it, int b, int scale_dt, uint32_t* __restrict__ hdr,
                                           bool dependent, uint32_t gen, const void* ph, ChainShared& sh) {
  using G = MfGeom<KIND>;
  constexpr int kT = WAVES * kWave;
  constexpr int D = kChainSlots / RB;
  auto& red = *reinterpret_cast<MfRed<WAVES, RB, 1>*>(sh.red);
  static_assert(sizeof(MfRed<WAVES, RB, 1>) <= sizeof(sh.red), "reduction image");

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const MfLane ln(lane);
  const int64_t N = it.n;
  const int64_t K = it.K;
  const int64_t n0 = static_cast<int64_t>(b - it.first_wg) * 8 * RB;
  const uint32_t tag = ((gen & 0x7fffu) + 1u) << 16;  // never 0; differs for consecutive generations

  const int64_t nseg_all = K / G::kSeg;
  const int64_t nseg = mf_uniform(wave < nseg_all ? (nseg_all - wave + WAVES - 1) / WAVES : 0);
  const int64_t kl = static_cast<int64_t>(G::kLaneK) * ln.slot();
  const uint8_t* w = static_cast<const uint8_t*>(it.w);  // loaded through a global view (MfMain)
  const uint8_t* wrow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int64_t row = std::min<int64_t>(n0 + 8 * rb + ln.r, N - 1);
    wrow[rb] = w + row * K * G::kEB + 16 * ln.slot();
  }
  MfXLds<KIND, 1> xs;
  xs.init(sh.xs, 1, static_cast<int>(K), 0, ln);
  floatx4 acc[RB][1];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb][0] = floatx4{0.f, 0.f, 0.f, 0.f};

  // The input. Its first batch of loads (64-bit: four external bf16 elements, or two tagged words) is issued
  // before the weight loads, so that reading it does not wait for them (loads complete in order per wave): a
  // workgroup whose input is already there pays no extra memory round trip. The rest of the input, and any word
  // still carrying an old tag, is read once the weight loads are in flight ("finish" below).
  const uint32_t* tin = dependent ? it.tag_in : nullptr;
  const bool external = it.tag_in == nullptr;
  const int64_t units = external ? K / 4 : K / 2;  // 64-bit loads for the whole input
  gptr<const uint64_t> src64 = as_global(static_cast<const uint64_t*>(external ? it.x : static_cast<const void*>(tin)));
  uint64_t pre[kGatherLoads];
#pragma unroll
  for (int u = 0; u < kGatherLoads; ++u) {
    const int64_t j = threadIdx.x + u * kT;
    pre[u] = 0;
    if (j < units && (external || tin != nullptr)) {
      if (external) pre[u] = src64[j];
      else pre[u] = ld_agent64(reinterpret_cast<const uint64_t*>(tin) + j);
    }
  }

  auto finish = [&]() {
    uint32_t* xs2 = reinterpret_cast<uint32_t*>(sh.xs);
    if (external) {
      for (int64_t j0 = 0; j0 < units; j0 += kGatherLoads * kT) {
#pragma unroll
        for (int u = 0; u < kGatherLoads; ++u) {
          const int64_t j = j0 + threadIdx.x + u * kT;
          if (j >= units) break;
          const uint64_t v = j0 == 0 ? pre[u] : src64[j];  // later batches: plain loads (after the weights)
          xs2[2 * j] = static_cast<uint32_t>(v);
          xs2[2 * j + 1] = static_cast<uint32_t>(v >> 32);
        }
      }
    } else {
      // Stale words in the first batch: once the producing stage is nearly done (its counter within the slack of
      // its workgroup count; one thread polls it), every thread re-reads its stale words until they carry the tag.
      bool stale = false;
#pragma unroll
      for (int u = 0; u < kGatherLoads; ++u) {
        const int64_t j = threadIdx.x + u * kT;
        if (j < units && (((static_cast<uint32_t>(pre[u]) & 0xffff0000u) != tag) ||
                          ((static_cast<uint32_t>(pre[u] >> 32) & 0xffff0000u) != tag)))
          stale = true;
      }
      bool wait = tin != nullptr;
      if (tin == nullptr) {  // an input from another item in a launch without hand-off: refused
        if (threadIdx.x == 0) st_agent(hdr + kHdrError, 1u);
      } else if (__syncthreads_or(stale)) {
        if (threadIdx.x == 0) {
          const uint32_t* ctr = hdr + kHdrCounters + it.dep_stage;
          const uint32_t need = static_cast<uint32_t>(it.dep_wgs);
          const uint32_t gate = need - std::min<uint32_t>(need - 1u, need / kSlackDiv);
          const uint32_t base = (gen - 1u) * need;
          long spins = 0;
          int ok = 1;
          while (ld_agent(ctr) - base < gate) {
            if (++spins > kSpinCounter) {
              st_agent(hdr + kHdrError, 1u);
              ok = 0;
              break;
            }
            __builtin_amdgcn_s_sleep(2);
          }
          sh.wait_ok = ok;
        }
        __syncthreads();
        wait = sh.wait_ok != 0;
        long spins = 0;
        while (wait && stale) {
          __builtin_amdgcn_s_sleep(1);
          stale = false;
#pragma unroll
          for (int u = 0; u < kGatherLoads; ++u) {
            const int64_t j = threadIdx.x + u * kT;
            const bool old = j < units && (((static_cast<uint32_t>(pre[u]) & 0xffff0000u) != tag) ||
                                           ((static_cast<uint32_t>(pre[u] >> 32) & 0xffff0000u) != tag));
            if (old) pre[u] = ld_agent64(reinterpret_cast<const uint64_t*>(tin) + j);
          }
#pragma unroll
          for (int u = 0; u < kGatherLoads; ++u) {
            const int64_t j = threadIdx.x + u * kT;
            if (j < units && (((static_cast<uint32_t>(pre[u]) & 0xffff0000u) != tag) ||
                              ((static_cast<uint32_t>(pre[u] >> 32) & 0xffff0000u) != tag)))
              stale = true;
          }
          if (stale && ++spins > kSpinWord) {
            st_agent(hdr + kHdrError, 1u);
            wait = false;
          }
        }
      }
      for (int64_t j0 = 0; j0 < units; j0 += kGatherLoads * kT) {
        if (j0 > 0) {
#pragma unroll
          for (int u = 0; u < kGatherLoads; ++u) {
            const int64_t j = j0 + threadIdx.x + u * kT;
            pre[u] = j < units && tin != nullptr ? ld_agent64(reinterpret_cast<const uint64_t*>(tin) + j) : 0;
          }
        }
#pragma unroll
        for (int u = 0; u < kGatherLoads; ++u) {
          const int64_t j = j0 + threadIdx.x + u * kT;
          if (j >= units) break;
          uint32_t w2[2] = {static_cast<uint32_t>(pre[u]), static_cast<uint32_t>(pre[u] >> 32)};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            long spins = 0;
            while (wait && (w2[h] & 0xffff0000u) != tag) {  // later batches (K above one batch)
              if (++spins > kSpinWord) {
                st_agent(hdr + kHdrError, 1u);
                wait = false;
                break;
              }
              __builtin_amdgcn_s_sleep(1);
              w2[h] = ld_agent(tin + 2 * j + h);
            }
          }
          xs2[j] = (w2[0] & 0xffffu) | (w2[1] << 16);
        }
      }
    }
    if (it.flags & BP_CHAIN_RENORM) {
      // the mean square in wave_sumsq's order (common.h): the renormalisation of the skinny kernel's prologue
      __syncthreads();
      const float tot = wave_sumsq_lds(sh.xs, static_cast<int>(K));
      __syncthreads();  // every wave has read the row before it is rewritten
      const float ms = tot / static_cast<float>(K);
      const float inv = ms > 0.f ? 1.f / sqrtf(ms) : 1.f;
      for (int64_t j = threadIdx.x; j < K; j += kT) sh.xs[j] = float_to_bf16_bits(bf16_bits_to_float(sh.xs[j]) * inv);
    }
    __syncthreads();
  };
  MfMain<KIND, 1, RB, D, true, false, MfXLds<KIND, 1>>::run(wrow, xs, ph, K, kl, wave, WAVES, nseg, acc, finish);

  mf_fold_halves<RB, 1>(acc);
  mf_store_red<WAVES, RB, 1>(red, acc, wave, lane);
  __syncthreads();
  gptr<uint16_t> y = as_global_mut(static_cast<uint16_t*>(it.y));
  uint32_t* tout = dependent ? it.tag_out : nullptr;
  for (int rr = threadIdx.x; rr < 8 * RB; rr += kT) {
    const int64_t n = n0 + rr;
    if (n >= N) continue;
    float t = mf_total<WAVES, RB, 1>(red, rr, 0);
    if constexpr (KIND == kInt8) t *= load_scale(it.scale, n, scale_dt);
    const uint16_t v = float_to_bf16_bits(t);
    if (y != nullptr) y[n] = v;
    if (tout != nullptr) st_agent(tout + n, tag | v);
  }
  if (tout == nullptr) return;
  // Report once every thread has issued its stores (not waiting for them to land: a consumer that reads a word
  // before it lands sees the old tag and reads it again).
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(hdr + kHdrCounters + it.stage, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Two workgroups of 8 waves per CU (at most 128 VGPRs): the weight tiles of both are in flight at once.
template <int KIND, int WAVES>
__global__ __launch_bounds__(WAVES * kWave, WAVES == 8 ? 2 : 1) void chain_kernel(const BpChainItem* __restrict__ items,
                                                              const int32_t* __restrict__ lut, int n_items,
                                                              int scale_dt, uint32_t* __restrict__ hdr, int dependent) {
  __shared__ __attribute__((aligned(16))) ChainShared sh;
  const int b = blockIdx.x;
  const BpChainItem& it = items[chain_item(items, lut, n_items, b)];
  const uint32_t gen = dependent ? ld_agent(hdr + kHdrGen) : 0u;
  // placeholder loads past a wave's last segment read the (cached) item table
  switch (it.rb) {
    case 1: chain_body<KIND, 1, WAVES>(it, b, scale_dt, hdr, dependent != 0, gen, items, sh); break;
    case 2: chain_body<KIND, 2, WAVES>(it, b, scale_dt, hdr, dependent != 0, gen, items, sh); break;
    default: chain_body<KIND, 4, WAVES>(it, b, scale_dt, hdr, dependent != 0, gen, items, sh); break;
  }
}

__global__ void chain_begin_kernel(uint32_t* hdr) {
  st_agent(hdr + kHdrGen, ld_agent(hdr + kHdrGen) + 1u);
}

using ChainFn = void (*)(const BpChainItem*, const int32_t*, int, int, uint32_t*, int);

ChainFn chain_pick(int wkind, int waves) {
  switch (wkind * 16 + waves) {
    case 0 * 16 + 2: return &chain_kernel<kBf16, 2>;
    case 0 * 16 + 4: return &chain_kernel<kBf16, 4>;
    case 0 * 16 + 8: return &chain_kernel<kBf16, 8>;
    case 1 * 16 + 2: return &chain_kernel<kInt8, 2>;
    case 1 * 16 + 4: return &chain_kernel<kInt8, 4>;
    case 1 * 16 + 8: return &chain_kernel<kInt8, 8>;
    default: return nullptr;
  }
}

}  // namespace
}  // namespace bp

extern "C" {

int bp_chain_supported(int wkind, int rb, int waves) {
  if (rb != 0 && rb != 1 && rb != 2 && rb != 4) return 0;
  return bp::chain_pick(wkind, waves) != nullptr ? 1 : 0;
}

size_t bp_chain_scratch_bytes(int num_stages) {
  if (num_stages < 0) return 0;
  return static_cast<size_t>(bp::kHdrCounters + num_stages) * sizeof(uint32_t);
}

int bp_chain_plan(BpChainItem* items, int num_items, int wkind, int rb, int waves, int32_t* lut, int lut_capacity) {
  if (items == nullptr || num_items <= 0 || !bp_chain_supported(wkind, rb, waves)) return BP_E_INVALID_ARG;
  const int64_t seg = wkind == bp::kBf16 ? 64 : 128;
  int64_t total = 0;
  int prev_stage = -1;
  for (int i = 0; i < num_items; ++i) {
    BpChainItem& it = items[i];
    if (it.w == nullptr || it.n <= 0 || it.K <= 0 || it.K > bp::kChainKMax || it.K % seg != 0) return BP_E_INVALID_ARG;
    if ((it.x == nullptr) == (it.tag_in == nullptr)) return BP_E_INVALID_ARG;  // exactly one input source
    if (it.stage < prev_stage || it.stage < 0) return BP_E_INVALID_ARG;        // items in stage order
    if (it.tag_in != nullptr && (it.dep_stage < 0 || it.dep_stage >= it.stage)) return BP_E_INVALID_ARG;
    if (reinterpret_cast<uintptr_t>(it.w) % 16 != 0) return BP_E_INVALID_ARG;
    // inputs are read four elements (external bf16) or two words (tagged) at a time
    if (reinterpret_cast<uintptr_t>(it.x) % 8 != 0 || reinterpret_cast<uintptr_t>(it.tag_in) % 8 != 0)
      return BP_E_INVALID_ARG;
    prev_stage = it.stage;
    it.rb = bp::chain_rb((it.K / seg + waves - 1) / waves, rb);
    it.first_wg = static_cast<int32_t>(total);
    total += (it.n + 8 * it.rb - 1) / (8 * it.rb);
    if (total > 0x7fffffff) return BP_E_INVALID_ARG;
  }
  // a consumer waits for every workgroup of the stage it reads
  for (int i = 0; i < num_items; ++i) {
    BpChainItem& it = items[i];
    if (it.tag_in == nullptr) {
      it.dep_wgs = 0;
      continue;
    }
    int64_t wgs = 0;
    for (int j = 0; j < num_items; ++j)
      if (items[j].stage == it.dep_stage) wgs += (items[j].n + 8 * items[j].rb - 1) / (8 * items[j].rb);
    if (wgs == 0) return BP_E_INVALID_ARG;  // reads a stage no item writes
    it.dep_wgs = static_cast<int32_t>(wgs);
  }
  const int64_t need = (total + 255) / 256;
  if (lut != nullptr) {
    if (lut_capacity < need) return BP_E_INVALID_ARG;
    int i = 0;
    for (int64_t c = 0; c < need; ++c) {
      while (i + 1 < num_items && items[i + 1].first_wg <= c * 256) ++i;
      lut[c] = i;
    }
  }
  return static_cast<int>(total);
}

int bp_chain_run(int wkind, int scale_dtype, const void* dev_items, const void* dev_lut, int num_items,
                 int total_wgs, int waves, void* scratch, int dependent, void* stream) {
  if (dev_items == nullptr || dev_lut == nullptr || num_items <= 0 || total_wgs <= 0) return BP_E_INVALID_ARG;
  if (wkind == bp::kInt8 && (scale_dtype < BP_DT_BF16 || scale_dtype > BP_DT_F32)) return BP_E_INVALID_ARG;
  if (scratch == nullptr) return BP_E_WORKSPACE;
  bp::ChainFn fn = bp::chain_pick(wkind, waves);
  if (fn == nullptr) return BP_E_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dependent) bp::chain_begin_kernel<<<1, 1, 0, st>>>(static_cast<uint32_t*>(scratch));
  fn<<<total_wgs, waves * bp::kWave, 0, st>>>(
      static_cast<const BpChainItem*>(dev_items), static_cast<const int32_t*>(dev_lut), num_items, scale_dtype,
      static_cast<uint32_t*>(scratch), dependent);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}

}  // extern "C"
