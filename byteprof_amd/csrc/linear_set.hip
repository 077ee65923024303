// Persistent kernel for a decode step's set of skinny linears at one activation row (batch-1 decode), gfx950.
//
// A decode step runs its linears as a chain of dependent stages: q|k|v share one input, o reads what attention made
// of v, gate|up read the attention block's output, down reads the MLP activation, the next layer's q|k|v read
// down's output, and the LM head reads the last layer's output. Launched one linear at a time, every stage pays
// a launch's fixed cost and HBM idles while a small launch ramps up and drains. This kernel runs the whole chain
// in one launch on one workgroup per CU and keeps the weight stream going across stage boundaries:
//
//   - compute waves (kSetCW per workgroup) own whole weight rows of every stage and stream them in 1 KiB
//     wave-wide chunks (16-byte non-temporal loads per lane) through a register ring of kSetRing chunks, so
//     kSetRing chunks per wave are in flight. Loads do not depend on activations, so a wave keeps
//     loading the next stage's rows while the stage's input is still being produced elsewhere on the chip;
//   - one sync wave per workgroup does all the cross-workgroup work, so the compute waves never wait for their
//     own outstanding loads: it gathers the stage's input vector into LDS (optionally renormalised to unit RMS)
//     and publishes the workgroup's results of the stage. Results travel as 32-bit words holding the bf16 value
//     and a per-launch tag, written and read with device-coherent (sc1) accesses: a reader that sees the current
//     tag in a word has its value, so publishing needs no release fence (an L2 writeback per workgroup and stage
//     costs more than the stage) and reading no acquire; a reader gathers its slice with LDS-DMA loads and waits
//     only for the rows it reads;
//   - inside the workgroup, LDS flags hand the input (xready) to the compute waves and the results (ydone)
//     back to the sync wave. Every wait is bounded: past a cap of polls the wave records an error flag in the
//     scratch words and stops waiting, so a launch always finishes.
//
// Nothing is reset between launches: launch g (counted by a launch counter every workgroup increments at the end)
// tags its words g % 65535 + 1, so the kernel can be replayed in a HIP graph with no memset. Per-row arithmetic matches the skinny kernels: bf16 (or
// exact int8 -> bf16) pairs through v_dot2_f32_bf16 into fp32, a fixed wave butterfly, the int8 scale on the fp32
// sum, round-to-nearest-even to bf16.
//
// Reference semantics per linear: byteprof/optim/skinny.py:36-90 (one-row product, bf16 / int8 modes); the set
// and its shapes: the decode-step linears that byteprof's OLMo-2 graph loop replays per token
// (byteprof/optim/olmo.py:164-215) and FINDINGS' "OLMo 2 16-block linear set".

#include "byteprof_amd.h"
#include "skinny_kernel.h"

namespace bp {
namespace {

#define BP_GLOBAL __attribute__((address_space(1)))
#define BP_LDS __attribute__((address_space(3)))
#define BP_CONST __attribute__((address_space(4)))

// Stage descriptors are read-only for the whole launch: read through the constant address space so that the
// wave-uniform reads become scalar loads.
typedef const BP_CONST BpSetStage* StageTable;
typedef const BP_GLOBAL u32x4* GlobalVec;

constexpr int kSetCW = 8;                           // compute waves per workgroup
constexpr int kSetThreads = (kSetCW + 1) * kWave;   // + one sync wave
constexpr int kSetKMax = 8192;                      // longest input vector (two bf16 buffers in LDS)
constexpr int kSetRowsMax = 2048;                   // rows of one stage per workgroup (fp32 results in LDS)
constexpr int kSetStagesMax = 256;                  // stages per set (row table in LDS)
constexpr int kSetRing = 32;                        // 1 KiB weight chunks in flight per compute wave
constexpr int kCtrWords = 32;                       // one 128-byte line per counter
constexpr uint32_t kSpinCapGlobal = 1u << 20;       // polls of a global counter before a wait gives up (~1 s)
constexpr uint32_t kSpinCapLds = 1u << 24;          // polls of an LDS flag before a wait gives up (~1 s)

struct SetLds {
  uint16_t x[2][kSetKMax];                // the stage's input vector, by stage parity
  uint32_t tin[kSetKMax];                 // tagged input words as gathered from the producing stage
  float y[2][kSetRowsMax];                // the workgroup's fp32 row sums, by stage parity
  float scale[2][kSetRowsMax];            // int8: the workgroup's row scales, by stage parity
  int32_t rows[kSetStagesMax][kSetCW + 1];  // stage s: wave i of this workgroup owns rows [rows[s][i], rows[s][i+1])
  int32_t tag_off[kSetStagesMax];         // word offset of stage s's tagged outputs in the scratch
  int xready;                             // stage s's input is in x[s & 1] once xready > s
  int ydone[2];                           // compute waves done with the stage of that parity
};
// More than half of the CU's 160 KiB of LDS: exactly one workgroup per CU, so the grid of one workgroup per CU is
// resident at once (the cross-workgroup waits rely on it).
static_assert(sizeof(SetLds) > 80 * 1024, "the set kernel must own its CU's LDS");
static_assert(sizeof(SetLds) <= 160 * 1024, "gfx950 LDS is 160 KiB per workgroup");

__device__ __forceinline__ int lds_load_relaxed(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Weight-chunk stream of one compute wave: its rows of every stage in stage order, each row in 1 KiB chunks.
// Every issue slot loads: once the stream has ended, slots re-read a valid chunk (`idle`) that nobody consumes,
// so the number of loads in flight is the same on every path and the compiler's wait counts stay exact.
template <int KIND>
struct Producer {
  int s;              // current stage (S: stream ended)
  int r, r1;          // current row, end of this wave's rows
  int c, C;           // chunk of the row, chunks per row
  int seg, seg_end;
  const BP_GLOBAL uint8_t* p;      // next chunk
  const BP_GLOBAL uint8_t* idle;   // a readable chunk for slots past the end
  int row_bytes;

  __device__ __forceinline__ void enter(StageTable st, const SetLds& L, int S, int wave, int from) {
    for (s = from; s < S; ++s) {
      r = uniform(L.rows[s][wave]);
      r1 = uniform(L.rows[s][wave + 1]);
      if (r < r1) break;
    }
    if (s >= S) {
      p = idle;
      return;
    }
    row_bytes = st[s].K * Layout<KIND>::kElemBytes;
    C = row_bytes >> 10;
    c = 0;
    seg = 0;
    int seg_begin = 0;
    while (st[s].seg_end[seg] <= r) seg_begin = st[s].seg_end[seg++];
    seg_end = st[s].seg_end[seg];
    p = (const BP_GLOBAL uint8_t*)(st[s].w[seg]) + static_cast<int64_t>(r - seg_begin) * row_bytes;
  }

  __device__ __forceinline__ void advance(StageTable st, const SetLds& L, int S, int wave) {
    if (s >= S) return;
    p += 1024;
    if (++c < C) return;
    c = 0;
    if (++r == r1) {
      enter(st, L, S, wave, s + 1);
    } else if (r == seg_end) {
      ++seg;
      seg_end = st[s].seg_end[seg];
      p = (const BP_GLOBAL uint8_t*)(st[s].w[seg]);
    }
  }

  __device__ __forceinline__ u32x4 issue(StageTable st, const SetLds& L, int S, int wave, int lane) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<GlobalVec>(p + lane * 16));
    advance(st, L, S, wave);
    return v;
  }
};

// Same chunks, same order, consumed: dot products against the stage input in LDS, one wave sum per row. The LDS
// chunk of the next item is read one item ahead. A wave visits only the stages where it owns rows; the sync wave
// counts those waves per stage.
template <int KIND>
struct Consumer {
  int s;
  int r, r1, row0;    // current row, end of this wave's rows, the workgroup's first row of the stage
  int c, C;
  float acc;
  bool failed;
  uint32_t xn[Layout<KIND>::kXDwords];  // input chunk of the current item

  __device__ __forceinline__ void load_x(const SetLds& L, int lane) {
    using Lay = Layout<KIND>;
    const u32x4* xs = reinterpret_cast<const u32x4*>(&L.x[s & 1][c * Lay::kChunk + lane * Lay::kEpl]);
#pragma unroll
    for (int q = 0; q < Lay::kXDwords / 4; ++q) {
      const u32x4 t = xs[q];
      xn[4 * q + 0] = t.x;
      xn[4 * q + 1] = t.y;
      xn[4 * q + 2] = t.z;
      xn[4 * q + 3] = t.w;
    }
  }

  // Moves to stage `from` or the next one with rows for this wave and waits (bounded) for its input in LDS.
  __device__ __forceinline__ void enter(StageTable st, SetLds& L, int S, int wave, int lane, int from) {
    for (s = from; s < S; ++s) {
      r = uniform(L.rows[s][wave]);
      r1 = uniform(L.rows[s][wave + 1]);
      if (r < r1) break;
    }
    if (s >= S) return;
    row0 = uniform(L.rows[s][0]);
    C = (st[s].K * Layout<KIND>::kElemBytes) >> 10;
    c = 0;
    acc = 0.f;
    uint32_t it = 0;
    while (!failed && lds_load_relaxed(&L.xready) <= s) {
      if (++it > kSpinCapLds) failed = true;
      __builtin_amdgcn_s_sleep(1);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    load_x(L, lane);
  }

  // Consumes one chunk (the stream's next item); false once every stage is done.
  __device__ __forceinline__ bool consume(const u32x4& wv, StageTable st, SetLds& L, int S, int wave, int lane) {
    if (s >= S) return false;
    acc = chunk_dot<KIND>(wv, xn, acc);
    if (++c == C) {
      const float tot = wave_sum_dpp(acc);
      if (lane == 0) L.y[s & 1][r - row0] = tot;
      acc = 0.f;
      c = 0;
      if (++r == r1) {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane == 0) __hip_atomic_fetch_add(&L.ydone[s & 1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        enter(st, L, S, wave, lane, s + 1);
        return true;
      }
    }
    load_x(L, lane);
    return true;
  }
};

// Scratch words: [0] launch counter (every workgroup adds 1 at the end of a launch), [kErrWord] error flag, then
// the tagged outputs of every stage (stage s at kTagWord + tag_off[s], N rounded up to 8 words): the bf16 bits in
// the low half, the launch's tag in the high half. A 32-bit store is seen whole or not at all, so a reader that
// finds the current launch's tag in a word has that launch's value: no fence, counter or flag is needed, and a
// reader waits only for the rows it reads.
constexpr int kErrWord = kCtrWords;
constexpr int kTagWord = 2 * kCtrWords;

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void record_error(uint32_t* scratch) { st_agent(&scratch[kErrWord], 1u); }

// Cache policy of the gather loads: sc1 (device scope), so they are served coherently across the XCDs' L2s.
constexpr int kDeviceScope = 16;

// Waits (bounded) until rows [e0, e0 + K) of an earlier stage carry this launch's tag and copies their bf16 values
// into xl. The tagged words come straight into LDS (global_load_lds_dwordx4, 1 KiB per wave instruction, no
// registers); chunks of 512 words with a word of an older tag are fetched again.
__device__ __forceinline__ void gather_input(const uint32_t* __restrict__ rows_t, int K, uint32_t tag, SetLds& L,
                                             uint16_t* xl, int lane, bool& failed, uint32_t* scratch) {
  const int nch = K / 512;
  uint32_t pending = (1u << nch) - 1u;  // wave-uniform; nch <= 16
  uint32_t it = 0;
  while (true) {
    for (int c = 0; c < nch; ++c) {
      if (!((pending >> c) & 1u)) continue;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        __builtin_amdgcn_global_load_lds((const BP_GLOBAL void*)(rows_t + c * 512 + h * 256 + lane * 4),
                                         (BP_LDS void*)&L.tin[c * 512 + h * 256], 16, 0, kDeviceScope);
    }
    __builtin_amdgcn_s_waitcnt(0);
    for (int c = 0; c < nch; ++c) {
      if (!((pending >> c) & 1u)) continue;
      const u32x4* tp = reinterpret_cast<const u32x4*>(&L.tin[c * 512 + lane * 8]);
      const u32x4 a = tp[0], b = tp[1];
      const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      bool ok = true;
#pragma unroll
      for (int e = 0; e < 8; ++e) ok = ok && (w[e] >> 16) == tag;
      if (__all(ok) || failed) {
        *reinterpret_cast<u32x4*>(xl + c * 512 + lane * 8) =
            u32x4{(w[0] & 0xffffu) | (w[1] << 16), (w[2] & 0xffffu) | (w[3] << 16), (w[4] & 0xffffu) | (w[5] << 16),
                  (w[6] & 0xffffu) | (w[7] << 16)};
        pending &= ~(1u << c);
      }
    }
    if (pending == 0u) break;
    if (++it > kSpinCapGlobal && !failed) {
      failed = true;
      record_error(scratch);
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// The workgroup's sync wave: inputs in, results out.
template <int KIND>
__device__ __forceinline__ void sync_wave(StageTable st, int S, uint32_t* __restrict__ scratch, SetLds& L,
                                          int scale_dt, int lane) {
  const int g = blockIdx.x, G = gridDim.x;
  // launch generation: every workgroup of the previous launches added 1 to the launch counter
  const uint32_t gen = ld_agent(&scratch[0]) / static_cast<uint32_t>(G);
  const uint32_t tag = gen % 65535u + 1u;  // 1..65535: a zeroed scratch holds no valid output
  uint32_t* tagged = scratch + kTagWord;
  bool failed = false;

  for (int s = 0; s < S; ++s) {
    const int K = st[s].K;
    const int row0 = L.rows[s][0];
    const int rows = L.rows[s][kSetCW] - row0;
    int active = 0;  // compute waves of this workgroup with rows in the stage
#pragma unroll
    for (int i = 0; i < kSetCW; ++i) active += L.rows[s][i] < L.rows[s][i + 1] ? 1 : 0;
    uint16_t* xl = L.x[s & 1];
    const int nch = K / 512;

    // 1. the input vector into LDS: published rows of an earlier stage, or an external vector
    const int ws = st[s].wait_stage;
    if (ws >= 0) {
      const int64_t e0 = (static_cast<const char*>(st[s].src) - static_cast<const char*>(st[ws].y)) / 2;
      gather_input(tagged + L.tag_off[ws] + e0, K, tag, L, xl, lane, failed, scratch);
    } else {
      const BP_GLOBAL uint16_t* src = (const BP_GLOBAL uint16_t*)(st[s].src);
      for (int c0 = 0; c0 < nch; c0 += 8) {
        u32x4 t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (c0 + j < nch) t[j] = *reinterpret_cast<GlobalVec>(src + (c0 + j) * 512 + lane * 8);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (c0 + j < nch) *reinterpret_cast<u32x4*>(xl + (c0 + j) * 512 + lane * 8) = t[j];
      }
    }
    // 2. optional unit-RMS scaling: mean square in a fixed order (per lane over its chunks, then a wave butterfly)
    if (st[s].renorm) {
      float ss = 0.f;
      for (int c0 = 0; c0 < nch; ++c0) {
        const u32x4 t = *reinterpret_cast<const u32x4*>(xl + c0 * 512 + lane * 8);
        const uint32_t d[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = bf16_bits_to_float(d[e] & 0xffffu), hi = bf16_bits_to_float(d[e] >> 16);
          ss += lo * lo;
          ss += hi * hi;
        }
      }
      float tot[1] = {ss};
      wave_transpose_reduce<1>(tot, lane);  // every lane holds the total
      const float ms = tot[0] / static_cast<float>(K);
      const float inv = ms > 0.f ? 1.f / sqrtf(ms) : 1.f;
      for (int c0 = 0; c0 < nch; ++c0) {
        u32x4* p = reinterpret_cast<u32x4*>(xl + c0 * 512 + lane * 8);
        const u32x4 t = *p;
        uint32_t d[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = float_to_bf16_bits(bf16_bits_to_float(d[e] & 0xffffu) * inv);
          const uint32_t hi = float_to_bf16_bits(bf16_bits_to_float(d[e] >> 16) * inv);
          d[e] = lo | (hi << 16);
        }
        *p = u32x4{d[0], d[1], d[2], d[3]};
      }
    }
    if (g == 0 && st[s].x_used != nullptr) {
      BP_GLOBAL uint16_t* xu = (BP_GLOBAL uint16_t*)(st[s].x_used);
      for (int c0 = 0; c0 < nch; ++c0)
        *reinterpret_cast<BP_GLOBAL u32x4*>(xu + c0 * 512 + lane * 8) =
            *reinterpret_cast<const u32x4*>(xl + c0 * 512 + lane * 8);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane == 0) __hip_atomic_store(&L.xready, s + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);

    // 3. while the compute waves work: int8 row scales of the stage into LDS
    if constexpr (KIND == kInt8) {
      for (int i = lane; i < rows; i += kWave) {
        const int row = row0 + i;
        int seg = 0, seg_begin = 0;
        while (st[s].seg_end[seg] <= row) seg_begin = st[s].seg_end[seg++];
        L.scale[s & 1][i] = load_scale(st[s].scale[seg], row - seg_begin, scale_dt);
      }
    }

    // 4. wait for the compute waves, publish the stage's rows (plain bf16 and tagged)
    {
      uint32_t it = 0;
      while (!failed && lds_load_relaxed(&L.ydone[s & 1]) < active) {
        if (++it > kSpinCapLds) {
          failed = true;
          record_error(scratch);
        }
        __builtin_amdgcn_s_sleep(1);
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    BP_GLOBAL uint16_t* y = (BP_GLOBAL uint16_t*)(st[s].y);
    uint32_t* ty = tagged + L.tag_off[s];
    for (int i = lane; i < rows; i += kWave) {
      float v = L.y[s & 1][i];
      if constexpr (KIND == kInt8) v *= L.scale[s & 1][i];
      const uint32_t bits = float_to_bf16_bits(v);
      y[row0 + i] = static_cast<uint16_t>(bits);
      st_agent(&ty[row0 + i], (tag << 16) | bits);
    }
    if (lane == 0) __hip_atomic_store(&L.ydone[s & 1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  if (lane == 0) __hip_atomic_fetch_add(&scratch[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int KIND>
__global__ __launch_bounds__(kSetThreads) void linear_set_kernel(const BpSetStage* __restrict__ stages, int S,
                                                                 uint32_t* __restrict__ scratch, int scale_dt) {
  __shared__ SetLds lds;
  StageTable st = (StageTable)(stages);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = uniform(threadIdx.x / kWave);
  // row table: wave i of workgroup g owns rows [u N / T, (u + 1) N / T) of every stage, u = g * CW + i
  const int64_t T = static_cast<int64_t>(gridDim.x) * kSetCW;
  for (int e = threadIdx.x; e < S * (kSetCW + 1); e += kSetThreads) {
    const int s = e / (kSetCW + 1), i = e % (kSetCW + 1);
    const int64_t u = static_cast<int64_t>(blockIdx.x) * kSetCW + i;
    lds.rows[s][i] = static_cast<int32_t>(u * st[s].N / T);
  }
  if (threadIdx.x == 0) {
    int32_t off = 0;
    for (int s = 0; s < S; ++s) {
      lds.tag_off[s] = off;
      off += (st[s].N + 7) & ~7;
    }
    lds.xready = 0;
    lds.ydone[0] = 0;
    lds.ydone[1] = 0;
  }
  __syncthreads();
  if (wave == kSetCW) {
    sync_wave<KIND>(st, S, scratch, lds, scale_dt, lane);
    return;
  }
  Producer<KIND> prod;
  prod.idle = (const BP_GLOBAL uint8_t*)(st[0].w[0]);
  prod.enter(st, lds, S, wave, 0);
  Consumer<KIND> cons;
  cons.failed = false;

  // Ring of kSetRing chunks: slot j is consumed, then reloaded with the chunk kSetRing items ahead, so every
  // consume finds exactly kSetRing - 1 younger loads in flight.
  u32x4 ring[kSetRing];
#pragma unroll
  for (int j = 0; j < kSetRing; ++j) ring[j] = prod.issue(st, lds, S, wave, lane);
  cons.enter(st, lds, S, wave, lane, 0);
  bool more = true;
  while (more) {
#pragma unroll
    for (int j = 0; j < kSetRing; ++j) {
      if (more) more = cons.consume(ring[j], st, lds, S, wave, lane);
      ring[j] = prod.issue(st, lds, S, wave, lane);  // unconditional: past the end it reloads the idle chunk
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
}

int set_validate(const BpSetStage* st, int S, int wkind, int G) {
  if (st == nullptr || S <= 0 || G <= 0) return BP_E_INVALID_ARG;
  if (S > kSetStagesMax) return BP_E_UNSUPPORTED;
  if (wkind != kBf16 && wkind != kInt8) return BP_E_UNSUPPORTED;
  if (G > 65536) return BP_E_UNSUPPORTED;
  const int64_t chunk = wkind == kBf16 ? 512 : 1024;
  int64_t words = 0;  // tagged outputs
  for (int s = 0; s < S; ++s) {
    const BpSetStage& a = st[s];
    if (a.src == nullptr || a.y == nullptr) return BP_E_INVALID_ARG;
    if (a.K <= 0 || a.K % chunk != 0 || a.K > kSetKMax) return BP_E_UNSUPPORTED;
    if (a.N <= 0 || static_cast<int64_t>(a.N) / G + 1 > kSetRowsMax) return BP_E_UNSUPPORTED;
    if (a.wait_stage < -1 || a.wait_stage >= s) return BP_E_INVALID_ARG;
    if (a.nseg < 1 || a.nseg > 4) return BP_E_INVALID_ARG;
    int32_t prev = 0;
    for (int j = 0; j < a.nseg; ++j) {
      if (a.seg_end[j] <= prev || a.w[j] == nullptr) return BP_E_INVALID_ARG;
      if (reinterpret_cast<uintptr_t>(a.w[j]) % 16 != 0) return BP_E_INVALID_ARG;
      if (wkind == kInt8 && a.scale[j] == nullptr) return BP_E_INVALID_ARG;
      prev = a.seg_end[j];
    }
    if (prev != a.N) return BP_E_INVALID_ARG;
    if (reinterpret_cast<uintptr_t>(a.src) % 16 != 0 || reinterpret_cast<uintptr_t>(a.y) % 16 != 0)
      return BP_E_INVALID_ARG;
    if (a.x_used != nullptr && reinterpret_cast<uintptr_t>(a.x_used) % 16 != 0) return BP_E_INVALID_ARG;
    if (a.wait_stage >= 0) {  // src must be K elements inside the waited-for stage's outputs
      const BpSetStage& p = st[a.wait_stage];
      const uintptr_t lo = reinterpret_cast<uintptr_t>(p.y), hi = lo + 2 * static_cast<uintptr_t>(p.N);
      const uintptr_t b = reinterpret_cast<uintptr_t>(a.src), e = b + 2 * static_cast<uintptr_t>(a.K);
      if (b < lo || e > hi) return BP_E_INVALID_ARG;
    }
    words += (a.N + 7) & ~7;
  }
  if (words > (int64_t{1} << 30)) return BP_E_UNSUPPORTED;
  return BP_OK;
}

int64_t scratch_words(const BpSetStage* st, int S, int G) {
  int64_t words = kTagWord;
  for (int s = 0; s < S; ++s) words += (st[s].N + 7) & ~7;
  return words;
}

}  // namespace
}  // namespace bp

extern "C" {

size_t bp_linear_set_scratch_bytes(const BpSetStage* stages, int num_stages, int num_workgroups) {
  if (stages == nullptr || num_stages <= 0 || num_workgroups <= 0) return 0;
  return static_cast<size_t>(bp::scratch_words(stages, num_stages, num_workgroups)) * sizeof(uint32_t);
}

int bp_linear_set_workgroups(int device) {
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
  return cus;
}

int bp_linear_set_validate(const BpSetStage* stages, int num_stages, int wkind, int num_workgroups) {
  return bp::set_validate(stages, num_stages, wkind, num_workgroups);
}

int bp_linear_set_run(int wkind, int scale_dtype, const BpSetStage* host_stages, const void* dev_stages,
                      int num_stages, void* scratch, size_t scratch_bytes, int num_workgroups, void* stream) {
  const int rc = bp::set_validate(host_stages, num_stages, wkind, num_workgroups);
  if (rc != BP_OK) return rc;
  if (dev_stages == nullptr || scratch == nullptr) return BP_E_INVALID_ARG;
  if (scratch_bytes < bp_linear_set_scratch_bytes(host_stages, num_stages, num_workgroups)) return BP_E_WORKSPACE;
  if (wkind == bp::kInt8 && (scale_dtype < BP_DT_BF16 || scale_dtype > BP_DT_F32)) return BP_E_INVALID_ARG;
  const auto* st = static_cast<const BpSetStage*>(dev_stages);
  auto* words = static_cast<uint32_t*>(scratch);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (wkind == bp::kBf16)
    bp::linear_set_kernel<bp::kBf16><<<num_workgroups, bp::kSetThreads, 0, s>>>(st, num_stages, words, scale_dtype);
  else
    bp::linear_set_kernel<bp::kInt8><<<num_workgroups, bp::kSetThreads, 0, s>>>(st, num_stages, words, scale_dtype);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}

}  // extern "C"
