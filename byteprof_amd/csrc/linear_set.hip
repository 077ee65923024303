// Persistent kernel for a decode step's set of skinny linears at one activation row (batch-1 decode), gfx950.
//
// A decode step runs its linears as a chain of dependent stages: q|k|v share one input, o reads what attention made
// of v, gate|up read the attention block's output, down reads the MLP activation, the next layer's q|k|v read
// down's output, and the LM head reads the last layer's output. Launched one linear at a time, every stage pays
// a launch's fixed cost and HBM idles while a small launch ramps up and drains. This kernel runs the whole chain
// in one launch on one workgroup per CU and keeps the weight stream going across stage boundaries:
//
//   - consumer waves (kSetCW per workgroup) own whole weight rows of every stage; each has a producer wave that
//     streams its rows in 1 KiB wave-wide chunks into an LDS ring (LDS-DMA loads, non-temporal). Loads do not
//     depend on activations, so the producers keep loading the next stage's rows while the stage's input is still
//     being produced elsewhere on the chip, and only they stall when the CU's outstanding loads are at capacity:
//     once a stage's input arrives, the consumers work through the landed ring at LDS speed;
//   - one sync wave per workgroup does all the cross-workgroup work, so the compute waves never wait for their
//     own outstanding loads: it gathers the stage's input vector into LDS (optionally renormalised to unit RMS)
//     and publishes the workgroup's results of the stage with device-coherent (sc1) stores and a per-workgroup
//     flag; readers poll the flags of the workgroups whose rows they read, then copy the rows into LDS with
//     device-scope LDS-DMA loads;
//   - inside the workgroup, LDS flags hand the input (xready) to the compute waves and the results (ydone)
//     back to the sync wave. Every wait is bounded: past a cap of polls the wave records an error flag in the
//     scratch words and stops waiting, so a launch always finishes.
//
// Nothing is reset between launches: launch g (counted by a launch counter every workgroup increments at the end)
// sets its flags to g + 1, so the kernel can be replayed in a HIP graph with no memset. Per-row arithmetic matches the skinny kernels: bf16 (or
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

constexpr int kSetCW = 4;                           // consumer waves per workgroup
constexpr int kSetPW = kSetCW;                      // producer waves: one per consumer
constexpr int kSetSyncWave = kSetCW + kSetPW;       // index of the sync wave
constexpr int kSetThreads = (kSetSyncWave + 1) * kWave;
constexpr int kSetKMax = 8192;                      // longest input vector (two bf16 buffers in LDS)
constexpr int kSetRowsMax = 1024;                   // rows of one stage per workgroup (fp32 results in LDS)
constexpr int kSetStagesMax = 128;                  // stages per set (row table in LDS)
constexpr int kSetSlots = 26;                       // 1 KiB LDS ring slots per consumer
constexpr int kSetLag = 12;                         // loads a producer keeps in flight before publishing them
constexpr int kSetPublish = 8;                      // chunks between two publications of the landed count
#ifndef BP_PUBMODE
#define BP_PUBMODE 16
#endif
constexpr int kCtrWords = 32;                       // one 128-byte line per counter
constexpr uint32_t kSpinCapGlobal = 1u << 20;       // polls of a global word before a wait gives up (~1 s)
constexpr uint32_t kSpinCapLds = 1u << 24;          // polls of an LDS word before a wait gives up (~1 s)

struct SetLds {
  alignas(16) uint8_t ring[kSetCW][kSetSlots][1024];  // weight chunks: producer i fills ring[i], consumer i drains it
  uint16_t x[2][kSetKMax];                // the stage's input vector, by stage parity
  float y[2][kSetRowsMax];                // the workgroup's fp32 row sums, by stage parity
  float scale[2][kSetRowsMax];            // int8: the workgroup's row scales, by stage parity
  int32_t rows[kSetStagesMax][kSetCW + 1];  // stage s: consumer i of this workgroup owns rows [rows[s][i], rows[s][i+1])
  int landed[kSetCW];                     // chunks of consumer i's stream in its ring (producer -> consumer)
  int consumed[kSetCW];                   // chunks consumer i has read out of its ring (consumer -> producer)
  int xready;                             // stage s's input is in x[s & 1] once xready > s
  int ydone[2];                           // consumer waves done with the stage of that parity
};
// More than half of the CU's 160 KiB of LDS: exactly one workgroup per CU, so the grid of one workgroup per CU is
// resident at once (the cross-workgroup waits rely on it).
static_assert(sizeof(SetLds) > 80 * 1024, "the set kernel must own its CU's LDS");
static_assert(sizeof(SetLds) <= 160 * 1024, "gfx950 LDS is 160 KiB per workgroup");

// s_waitcnt immediate that waits for at most N vector memory operations in flight (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
template <int N>
constexpr int waitcnt_vm() {
  return (N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8);
}

__device__ __forceinline__ int lds_load_relaxed(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Weight-chunk stream of one consumer: its rows of every stage in stage order, each row in 1 KiB chunks.
template <int KIND>
struct Cursor {
  int s;              // current stage (S: stream ended)
  int r, r1;          // current row, end of the consumer's rows
  int c, C;           // chunk of the row, chunks per row
  int seg, seg_end;
  const BP_GLOBAL uint8_t* p;  // next chunk
  int row_bytes;

  __device__ __forceinline__ void enter(StageTable st, const SetLds& L, int S, int who, int from) {
    for (s = from; s < S; ++s) {
      r = uniform(L.rows[s][who]);
      r1 = uniform(L.rows[s][who + 1]);
      if (r < r1) break;
    }
    if (s >= S) return;
    row_bytes = st[s].K * Layout<KIND>::kElemBytes;
    C = row_bytes >> 10;
    c = 0;
    seg = 0;
    int seg_begin = 0;
    while (st[s].seg_end[seg] <= r) seg_begin = st[s].seg_end[seg++];
    seg_end = st[s].seg_end[seg];
    p = (const BP_GLOBAL uint8_t*)(st[s].w[seg]) + static_cast<int64_t>(r - seg_begin) * row_bytes;
  }

  __device__ __forceinline__ void advance(StageTable st, const SetLds& L, int S, int who) {
    p += 1024;
    if (++c < C) return;
    c = 0;
    if (++r == r1) {
      enter(st, L, S, who, s + 1);
    } else if (r == seg_end) {
      ++seg;
      seg_end = st[s].seg_end[seg];
      p = (const BP_GLOBAL uint8_t*)(st[s].w[seg]);
    }
  }
};

// Cache policy of the weight stream: nt (streamed once, not kept in the caches).
constexpr int kStreamPolicy = 2;

// Producer wave i: copies consumer i's chunks into its LDS ring with LDS-DMA loads (global_load_lds_dwordx4,
// 1 KiB per wave instruction, no registers). A load instruction stalls its wave while the CU's outstanding requests
// are at capacity; only this wave stalls, so the consumer keeps reading landed chunks at LDS speed. Loads complete
// in order: after each load the producer waits until at most kSetLag are in flight and publishes the count that
// has landed. When the ring is full (its consumer is waiting for a stage's input) it publishes everything and
// waits for a free slot, so a consumer that resumes finds the whole ring landed.
template <int KIND>
__device__ __forceinline__ void producer_wave(StageTable st, SetLds& L, int S, int who, int lane) {
  Cursor<KIND> cur;
  cur.enter(st, L, S, who, 0);
  int n = 0, limit = kSetSlots;  // chunks issued; chunks that fit the ring as last seen
  bool failed = false;
  while (cur.s < S) {
    if (n >= limit) {  // ring full as last seen: publish everything, then wait for the consumer
      __builtin_amdgcn_s_waitcnt(waitcnt_vm<0>());
      if (lane == 0) __hip_atomic_store(&L.landed[who], n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      uint32_t it = 0;
      while (!failed && n >= (limit = lds_load_relaxed(&L.consumed[who]) + kSetSlots)) {
        if (++it > kSpinCapLds) failed = true;
        __builtin_amdgcn_s_sleep(1);
      }
      if (failed) break;
    }
    __builtin_amdgcn_global_load_lds((const BP_GLOBAL void*)(cur.p + lane * 16),
                                     (BP_LDS void*)&L.ring[who][n % kSetSlots][0], 16, 0, kStreamPolicy);
    cur.advance(st, L, S, who);
    ++n;
#if BP_PUBMODE == 0
    if (n > kSetLag) __builtin_amdgcn_s_waitcnt(waitcnt_vm<kSetLag>());
    // An LDS access of this wave waits for the LDS writes of its loads in flight, so the producer touches LDS
    // every kSetPublish chunks only: it publishes what has landed and refreshes its view of the consumer.
    if (n % kSetPublish == 0) {
      if (lane == 0 && n > kSetLag)
        __hip_atomic_store(&L.landed[who], n - kSetLag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      limit = lds_load_relaxed(&L.consumed[who]) + kSetSlots;
    }
#else
    if (n % BP_PUBMODE == 0) {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm<0>());
      if (lane == 0) __hip_atomic_store(&L.landed[who], n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      limit = lds_load_relaxed(&L.consumed[who]) + kSetSlots;
    }
#endif
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm<0>());
  if (lane == 0) __hip_atomic_store(&L.landed[who], n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Consumer wave i: the same chunks in the same order, read from its LDS ring once landed: dot products against
// the stage input in LDS, one wave sum per row. Chunks are taken in groups of GS of one row (GS divides the
// chunks per row): one poll of the landed count, all of the group's LDS reads in flight together, one release of
// its ring slots. A consumer visits only the stages where it owns rows; the sync wave counts those per stage.
template <int KIND>
struct Consumer {
  int s;
  int r, r1, row0;    // current row, end of this consumer's rows, the workgroup's first row of the stage
  int c, C;
  int n, seen;        // chunks consumed; chunks known to have landed
  float acc;
  bool failed;

  // Moves to stage `from` or the next one with rows for this consumer and waits (bounded) for its input in LDS.
  __device__ __forceinline__ void enter(StageTable st, SetLds& L, int S, int who, int from) {
    for (s = from; s < S; ++s) {
      r = uniform(L.rows[s][who]);
      r1 = uniform(L.rows[s][who + 1]);
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
  }

  // GS chunks of the current row. RESIDENT: the row is exactly these GS chunks and xr already holds the stage's
  // input chunks (loaded once per stage), so only the weights are read from LDS.
  template <int GS, bool RESIDENT>
  __device__ __forceinline__ void group(StageTable st, SetLds& L, int S, int who, int lane,
                                        uint32_t (&xr)[4][Layout<KIND>::kXDwords]) {
    using Lay = Layout<KIND>;
    uint32_t it = 0;
    while (seen < n + GS && !failed) {
      seen = lds_load_relaxed(&L.landed[who]);
      if (seen >= n + GS) break;
      if (++it > kSpinCapLds) failed = true;
      __builtin_amdgcn_s_sleep(0);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    u32x4 w[GS];
    uint32_t xv[GS][Lay::kXDwords];
    int slot = n % kSetSlots;
#pragma unroll
    for (int j = 0; j < GS; ++j) {
      w[j] = *reinterpret_cast<const u32x4*>(&L.ring[who][slot][lane * 16]);
      slot = slot + 1 == kSetSlots ? 0 : slot + 1;
      if constexpr (!RESIDENT) {
        const u32x4* xs = reinterpret_cast<const u32x4*>(&L.x[s & 1][(c + j) * Lay::kChunk + lane * Lay::kEpl]);
#pragma unroll
        for (int q = 0; q < Lay::kXDwords / 4; ++q) {
          const u32x4 t = xs[q];
          xv[j][4 * q + 0] = t.x;
          xv[j][4 * q + 1] = t.y;
          xv[j][4 * q + 2] = t.z;
          xv[j][4 * q + 3] = t.w;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < GS; ++j) acc = chunk_dot<KIND>(w[j], RESIDENT ? xr[j] : xv[j], acc);
    n += GS;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane == 0) __hip_atomic_store(&L.consumed[who], n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    c += GS;
    if (c == C) {
      const float tot = wave_sum_dpp(acc);
      if (lane == 0) L.y[s & 1][r - row0] = tot;
      acc = 0.f;
      c = 0;
      if (++r == r1) {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane == 0) __hip_atomic_fetch_add(&L.ydone[s & 1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        enter(st, L, S, who, s + 1);
      }
    }
  }

  __device__ __forceinline__ void run(StageTable st, SetLds& L, int S, int who, int lane) {
    using Lay = Layout<KIND>;
    uint32_t xr[4][Lay::kXDwords];
    enter(st, L, S, who, 0);
    while (s < S) {
      if (C == 4 || C == 2) {  // whole rows per group: the stage's input chunks stay in registers
        const int stage = s;
        for (int j = 0; j < C; ++j) {
          const u32x4* xs = reinterpret_cast<const u32x4*>(&L.x[s & 1][j * Lay::kChunk + lane * Lay::kEpl]);
#pragma unroll
          for (int q = 0; q < Lay::kXDwords / 4; ++q) {
            const u32x4 t = xs[q];
            // static register index: j is 0..3 (unrolled by the select below)
            if (j == 0) { xr[0][4 * q + 0] = t.x; xr[0][4 * q + 1] = t.y; xr[0][4 * q + 2] = t.z; xr[0][4 * q + 3] = t.w; }
            if (j == 1) { xr[1][4 * q + 0] = t.x; xr[1][4 * q + 1] = t.y; xr[1][4 * q + 2] = t.z; xr[1][4 * q + 3] = t.w; }
            if (j == 2) { xr[2][4 * q + 0] = t.x; xr[2][4 * q + 1] = t.y; xr[2][4 * q + 2] = t.z; xr[2][4 * q + 3] = t.w; }
            if (j == 3) { xr[3][4 * q + 0] = t.x; xr[3][4 * q + 1] = t.y; xr[3][4 * q + 2] = t.z; xr[3][4 * q + 3] = t.w; }
          }
        }
        if (C == 4) {
          while (s == stage) group<4, true>(st, L, S, who, lane, xr);
        } else {
          while (s == stage) group<2, true>(st, L, S, who, lane, xr);
        }
      } else if ((C & 3) == 0) {
        group<4, false>(st, L, S, who, lane, xr);
      } else if ((C & 1) == 0) {
        group<2, false>(st, L, S, who, lane, xr);
      } else {
        group<1, false>(st, L, S, who, lane, xr);
      }
    }
  }
};

// Scratch words: [0] launch counter (every workgroup adds 1 at the end of a launch), [kErrWord] error flag, then
// S x G publish flags from kFlagWord: flag[s][g] = the launch's tag once workgroup g's rows of stage s are visible
// device-wide. A producer stores its rows with device-scope (sc1, write-through) stores, waits until they are
// acknowledged, then stores its flag; a reader polls the flags of the workgroups that produce the rows it reads
// (one word each, all of a poll's loads in flight together) and then reads the rows with device-scope loads. Both
// sides use device-coherent accesses for the rows, so no L2 writeback or invalidate is needed (a release fence
// per workgroup and stage costs more than a stage), and a reader waits only for the rows it reads.
constexpr int kErrWord = kCtrWords;
constexpr int kFlagWord = 2 * kCtrWords;

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent16(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void record_error(uint32_t* scratch) { st_agent(&scratch[kErrWord], 1u); }

// Cache policy of the gather loads: sc1 (device scope), so they are served coherently across the XCDs' L2s.
constexpr int kDeviceScope = 16;

// The workgroup that computes row r of a stage of N rows (workgroup g owns rows [g N / G, (g + 1) N / G)).
__device__ __forceinline__ int owner_of(int64_t r, int64_t N, int G) {
  return static_cast<int>(((r + 1) * G + N - 1) / N) - 1;
}

// Waits (bounded) until every workgroup in [g_lo, g_hi] has set its flag to `tag`: one load per workgroup per
// poll, all of a poll's loads in flight together.
__device__ __forceinline__ void wait_flags(const uint32_t* __restrict__ flags, int g_lo, int g_hi, uint32_t tag,
                                           int lane, bool& failed, uint32_t* scratch) {
  uint32_t it = 0;
  while (!failed) {
    bool ok = true;
    for (int g0 = g_lo; g0 <= g_hi; g0 += 4 * kWave) {
      uint32_t f[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) f[i] = ld_agent(&flags[min(g0 + i * kWave + lane, g_hi)]);
#pragma unroll
      for (int i = 0; i < 4; ++i) ok = ok && f[i] == tag;
    }
    if (__all(ok)) return;
    if (++it > kSpinCapGlobal) {
      failed = true;
      record_error(scratch);
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Copies K published bf16 values into xl with device-scope LDS-DMA loads (global_load_lds_dwordx4: 1 KiB, one
// 512-element chunk of the LDS layout, per wave instruction, no registers).
__device__ __forceinline__ void gather_rows(const uint16_t* __restrict__ src, int K, uint16_t* xl, int lane) {
  for (int c = 0; c < K / 512; ++c)
    __builtin_amdgcn_global_load_lds((const BP_GLOBAL void*)(src + c * 512 + lane * 8), (BP_LDS void*)(xl + c * 512),
                                     16, 0, kDeviceScope);
  __builtin_amdgcn_s_waitcnt(0);
}

// The workgroup's sync wave: inputs in, results out.
template <int KIND>
__device__ __forceinline__ void sync_wave(StageTable st, int S, uint32_t* __restrict__ scratch, SetLds& L,
                                          int scale_dt, int lane) {
  const int g = blockIdx.x, G = gridDim.x;
  // launch generation: every workgroup of the previous launches added 1 to the launch counter
  const uint32_t gen = ld_agent(&scratch[0]) / static_cast<uint32_t>(G);
  const uint32_t tag = gen + 1u;  // never 0, the value of a zeroed scratch (wraps after 2^32 - 1 launches)
  uint32_t* flags = scratch + kFlagWord;
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
      const int64_t Nw = st[ws].N;
      wait_flags(flags + static_cast<int64_t>(ws) * G, owner_of(e0, Nw, G), owner_of(e0 + K - 1, Nw, G), tag, lane,
                 failed, scratch);
      gather_rows(static_cast<const uint16_t*>(st[s].src), K, xl, lane);
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
    // 2. optional unit-RMS scaling: mean square in a fixed order (per lane over its chunks, then a wave butterfly).
    //    Chunks are taken four at a time so that their LDS reads are in flight together.
    if (st[s].renorm) {
      float ss = 0.f;
      for (int c0 = 0; c0 < nch; c0 += 4) {
        u32x4 t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          t[j] = c0 + j < nch ? *reinterpret_cast<const u32x4*>(xl + (c0 + j) * 512 + lane * 8) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t d[4] = {t[j].x, t[j].y, t[j].z, t[j].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float lo = bf16_bits_to_float(d[e] & 0xffffu), hi = bf16_bits_to_float(d[e] >> 16);
            ss += lo * lo;
            ss += hi * hi;
          }
        }
      }
      float tot[1] = {ss};
      wave_transpose_reduce<1>(tot, lane);  // every lane holds the total
      const float ms = tot[0] / static_cast<float>(K);
      const float inv = ms > 0.f ? 1.f / sqrtf(ms) : 1.f;
      for (int c0 = 0; c0 < nch; c0 += 4) {
        u32x4 t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (c0 + j < nch) t[j] = *reinterpret_cast<const u32x4*>(xl + (c0 + j) * 512 + lane * 8);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (c0 + j >= nch) continue;
          uint32_t d[4] = {t[j].x, t[j].y, t[j].z, t[j].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t lo = float_to_bf16_bits(bf16_bits_to_float(d[e] & 0xffffu) * inv);
            const uint32_t hi = float_to_bf16_bits(bf16_bits_to_float(d[e] >> 16) * inv);
            d[e] = lo | (hi << 16);
          }
          *reinterpret_cast<u32x4*>(xl + (c0 + j) * 512 + lane * 8) = u32x4{d[0], d[1], d[2], d[3]};
        }
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

    // 4. wait for the compute waves, publish the stage's rows
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
    // rows with device-scope stores; once they are acknowledged, the flag
    uint16_t* y = static_cast<uint16_t*>(st[s].y);
    for (int i = lane; i < rows; i += kWave) {
      float v = L.y[s & 1][i];
      if constexpr (KIND == kInt8) v *= L.scale[s & 1][i];
      st_agent16(&y[row0 + i], float_to_bf16_bits(v));
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (lane == 0) {
      st_agent(&flags[static_cast<int64_t>(s) * G + g], tag);
      __hip_atomic_store(&L.ydone[s & 1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
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
  // row table: consumer i of workgroup g owns rows [u N / T, (u + 1) N / T) of every stage, u = g * CW + i
  const int64_t T = static_cast<int64_t>(gridDim.x) * kSetCW;
  for (int e = threadIdx.x; e < S * (kSetCW + 1); e += kSetThreads) {
    const int s = e / (kSetCW + 1), i = e % (kSetCW + 1);
    const int64_t u = static_cast<int64_t>(blockIdx.x) * kSetCW + i;
    lds.rows[s][i] = static_cast<int32_t>(u * st[s].N / T);
  }
  if (threadIdx.x < kSetCW) {
    lds.landed[threadIdx.x] = 0;
    lds.consumed[threadIdx.x] = 0;
  }
  if (threadIdx.x == 0) {
    lds.xready = 0;
    lds.ydone[0] = 0;
    lds.ydone[1] = 0;
  }
  __syncthreads();
  if (wave == kSetSyncWave) {
    sync_wave<KIND>(st, S, scratch, lds, scale_dt, lane);
  } else if (wave >= kSetCW) {
    producer_wave<KIND>(st, lds, S, wave - kSetCW, lane);
  } else {
    Consumer<KIND> cons;
    cons.failed = false;
    cons.n = 0;
    cons.seen = 0;
    cons.run(st, lds, S, wave, lane);
  }
}

int set_validate(const BpSetStage* st, int S, int wkind, int G) {
  if (st == nullptr || S <= 0 || G <= 0) return BP_E_INVALID_ARG;
  if (S > kSetStagesMax) return BP_E_UNSUPPORTED;
  if (wkind != kBf16 && wkind != kInt8) return BP_E_UNSUPPORTED;
  if (G > 65536) return BP_E_UNSUPPORTED;
  const int64_t chunk = wkind == kBf16 ? 512 : 1024;
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
  }
  return BP_OK;
}

int64_t scratch_words(int S, int G) { return kFlagWord + static_cast<int64_t>(S) * G; }

}  // namespace
}  // namespace bp

extern "C" {

size_t bp_linear_set_scratch_bytes(const BpSetStage* stages, int num_stages, int num_workgroups) {
  if (stages == nullptr || num_stages <= 0 || num_workgroups <= 0) return 0;
  return static_cast<size_t>(bp::scratch_words(num_stages, num_workgroups)) * sizeof(uint32_t);
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
