// Persistent kernel for a decode step's set of skinny linears at one activation row (batch-1 decode), gfx950.
//
// A decode step runs its linears as a chain of dependent stages: q|k|v share one input, o reads what attention made
// of v, gate|up read the attention block's output, down reads the MLP activation, the next layer's q|k|v read
// down's output, and the LM head reads the last layer's output. Launched one linear at a time, every stage pays
// a launch's fixed cost and HBM idles while a small launch ramps up and drains. This kernel runs the whole chain
// in one launch on one workgroup per CU and keeps the weight stream going across stage boundaries. A workgroup
// has three kinds of waves:
//
//   - consumer waves (kSetCW) own whole weight rows of every stage: they take their rows' 1 KiB weight chunks
//     from an LDS ring, dot them with the stage input in LDS (v_dot2_f32_bf16, fp32), sum each row over the wave
//     and publish it;
//   - producer waves (one per consumer) stream the consumer's chunks with non-temporal 16-byte loads through a
//     small register ring into its LDS ring, publishing each chunk as it lands. Loads do not depend on
//     activations, so producers keep loading the next stages' rows while a stage's input is still being computed
//     elsewhere on the chip; a load instruction stalls its wave while the CU's outstanding requests are at
//     capacity, and only producers stall, so when a stage's input arrives the consumers work through the landed
//     ring at LDS speed;
//   - one sync wave gathers each stage's input vector into LDS (optionally renormalised to unit RMS) and hands it
//     to the consumers.
//
// Rows travel between workgroups as 32-bit words: the bf16 value in the low half, a per-launch tag in the high
// half, written by the consumer that computed the row with a device-scope (sc1, write-through) store. A 32-bit
// store is seen whole or not at all, so a reader that finds the current tag in a word has that launch's value: no
// fence, counter or flag is needed (a release fence per workgroup and stage costs more than a stage), and a reader
// waits only for the rows it reads. The sync wave starts reading a stage's input once its own consumers have
// finished the producing stage, with device-scope LDS-DMA loads, and reads again the chunks still carrying an
// older tag. Every wait is bounded: past a cap of polls the wave records an error flag in the scratch and stops
// waiting, so a launch always finishes.
//
// Nothing is reset between launches: launch g (counted by a launch counter every workgroup increments at the end)
// tags its words g % 65535 + 1, so the kernel can be replayed in a HIP graph with no memset. Per-row arithmetic
// matches the skinny kernels: bf16 (or exact int8 -> bf16) pairs through v_dot2_f32_bf16 into fp32, a fixed wave
// reduction order, the int8 scale on the fp32 sum, round-to-nearest-even to bf16.
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
constexpr int kSetTin = 4096;                       // tagged input words gathered per round (16 KiB)
constexpr int kSetRowsMax = 512;                    // rows of one stage per workgroup (int8 scales in LDS)
constexpr int kSetStagesMax = 96;                   // stages per set (tables in LDS)
constexpr int kSetSlots = 26;                       // 1 KiB LDS ring slots per consumer
constexpr int kSetInflight = 12;                    // weight chunks a producer keeps in flight (registers)
constexpr int kWordsHeader = 64;                    // scratch: launch counter (word 0), error flag (word 32)
constexpr int kErrWord = 32;
constexpr uint32_t kSpinCapGlobal = 1u << 20;       // polls of global memory before a wait gives up (~1 s)
constexpr uint32_t kSpinCapLds = 1u << 24;          // polls of an LDS word before a wait gives up (~1 s)

struct SetLds {
  alignas(16) uint8_t ring[kSetCW][kSetSlots][1024];  // weight chunks: producer i fills ring[i], consumer i drains it
  alignas(16) uint16_t x[2][kSetKMax];    // the stage's input vector, by stage parity
  alignas(16) uint32_t tin[kSetTin];      // tagged input words as gathered
  float scale[2][kSetRowsMax];            // int8: the workgroup's row scales, by stage parity
  int32_t rows[kSetStagesMax][kSetCW + 1];  // stage s: consumer i owns rows [rows[s][i], rows[s][i+1])
  int32_t tag_off[kSetStagesMax];         // word offset of stage s's tagged rows after the scratch header
  int done[kSetStagesMax];                // consumers of this workgroup done with stage s
  int landed[kSetCW];                     // chunks of consumer i's stream in its ring (producer -> consumer)
  int consumed[kSetCW];                   // chunks consumer i has read out of its ring (consumer -> producer)
  int xready;                             // stage s's input is in x[s & 1] once xready > s
  uint32_t tag;                           // this launch's tag
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

// s_waitcnt lgkmcnt(0), vector memory and export counts left at their maxima. Ends a path that issued scalar loads,
// so that no scalar load is pending where it joins the common path (lgkmcnt also counts LDS operations, and the
// only wait the compiler can place for an out-of-order scalar load at a join is lgkmcnt(0), which would make every
// chunk of the common path wait for its own LDS writes).
constexpr int kWaitLgkm0 = 0xF | (0x3 << 14) | (0x7 << 4);

__device__ __forceinline__ int lds_load_relaxed(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_store_relaxed(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void record_error(uint32_t* scratch) { st_agent(&scratch[kErrWord], 1u); }

// Cache policy of the gathers of published rows: device scope (sc1), served coherently across the XCDs' L2s.
constexpr int kDeviceScope = 16;

// Weight-chunk stream of one consumer: its rows of every stage in stage order, each row in 1 KiB chunks. The rows
// of one weight segment are contiguous in memory, so the stream is a sequence of contiguous runs (the consumer's
// rows of a stage within one segment): the common step is one 64-bit add and one count, and the stage table is read
// only where a run ends.
template <int KIND>
struct Cursor {
  int s;              // current stage (S: stream ended)
  int r, r1;          // first row after the current run, end of the consumer's rows in stage s
  int seg;            // segment of the current run
  int left;           // chunks left in the current run
  const BP_GLOBAL uint8_t* p;  // the next chunk; once the stream has ended, its first chunk (loads stay in bounds)
  const BP_GLOBAL uint8_t* first;

  // The run of rows r .. min(r1, end of segment seg) - 1.
  __device__ __forceinline__ void start_run(StageTable st, int seg_begin) {
    const int row_bytes = st[s].K * Layout<KIND>::kElemBytes;
    const int run_end = min(r1, st[s].seg_end[seg]);
    left = (run_end - r) * (row_bytes >> 10);
    p = (const BP_GLOBAL uint8_t*)(st[s].w[seg]) + static_cast<int64_t>(r - seg_begin) * row_bytes;
    r = run_end;
    // the stage-table values in registers here, so that no scalar load is pending where the common path resumes
    asm volatile("" ::"s"(p), "s"(left));
  }

  __device__ __forceinline__ void enter(StageTable st, const SetLds& L, int S, int who, int from) {
    for (s = from; s < S; ++s) {
      r = uniform(L.rows[s][who]);
      r1 = uniform(L.rows[s][who + 1]);
      if (r < r1) break;
    }
    if (s >= S) {
      p = first;
      return;
    }
    seg = 0;
    int seg_begin = 0;
    while (st[s].seg_end[seg] <= r) seg_begin = st[s].seg_end[seg++];
    start_run(st, seg_begin);
  }

  __device__ __forceinline__ void advance(StageTable st, const SetLds& L, int S, int who) {
    p += 1024;
    if (__builtin_expect(--left > 0, 1)) return;
    if (r == r1) {
      enter(st, L, S, who, s + 1);
    } else {  // r is the first row of segment seg + 1
      ++seg;
      start_run(st, r);
    }
  }
};

// Producer wave `who`: copies its consumer's chunks into the consumer's LDS ring. Chunks travel through a ring of
// kSetInflight registers: the producer waits for its oldest load, writes that chunk into the LDS ring, publishes
// it at once (one LDS word), and loads the next chunk into the freed registers. Exactly kSetInflight loads are
// always in flight (past the end of its stream the producer re-reads its first chunk), so each wait is for the
// oldest load only. Four producers keep 4 * kSetInflight KiB in flight per CU, below the CU's capacity, so the
// sync wave's loads are not queued behind the weight stream. When the LDS ring is full (its consumer is waiting
// for a stage's input) the producer waits for a free slot with its loads still in flight.
template <int KIND>
__device__ __forceinline__ void producer_wave(StageTable st, SetLds& L, int S, int who, int lane,
                                              uint32_t* scratch) {
  Cursor<KIND> cur;
  cur.first = nullptr;
  cur.enter(st, L, S, who, 0);
  if (cur.s >= S) return;  // no rows in any stage: the consumer has none either
  cur.first = cur.p;
  // a 32-bit lane offset on a wave-uniform base: the loads take the scalar-base form (saddr + voffset), with no
  // per-chunk vector address arithmetic on the SIMD the producer shares with its consumer
  const uint32_t lane_off = static_cast<uint32_t>(lane) * 16u;
  u32x4 buf[kSetInflight];
  int issued = 0;
#pragma unroll
  for (int j = 0; j < kSetInflight; ++j) {
    const bool real = cur.s < S;
    buf[j] = __builtin_nontemporal_load((const BP_GLOBAL u32x4*)(cur.p + lane_off));
    if (real) {
      cur.advance(st, L, S, who);
      ++issued;
    }
  }
  int n = 0, slot = 0, limit = kSetSlots;  // chunks written to the ring; ring slot of chunk n; chunks that fit
  bool failed = false;
  while (n < issued) {
#pragma unroll
    for (int j = 0; j < kSetInflight; ++j) {
      if (n < issued) {
        if (n >= limit) {
          uint32_t it = 0;
          while (!failed && n >= (limit = uniform(lds_load_relaxed(&L.consumed[who])) + kSetSlots)) {
            if (++it > kSpinCapLds) {
              failed = true;
              record_error(scratch);
            }
            __builtin_amdgcn_s_sleep(1);
          }
          if (failed) limit = n + kSetSlots;  // stop waiting; the launch's results are flagged invalid
        }
        *reinterpret_cast<u32x4*>(&L.ring[who][slot][lane * 16]) = buf[j];
        ++n;
        slot = slot + 1 == kSetSlots ? 0 : slot + 1;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane == 0) lds_store_relaxed(&L.landed[who], n);
      }
      const bool real = cur.s < S;
      buf[j] = __builtin_nontemporal_load((const BP_GLOBAL u32x4*)(cur.p + lane_off));
      if (real) {
        cur.advance(st, L, S, who);
        ++issued;
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm<0>());
}

// Consumer wave `who`: the same chunks in the same order, read from its ring once landed, in groups of GS chunks
// of one row (GS divides the chunks per row): one poll of the landed count, all of the group's LDS reads in flight
// together, one release of the group's ring slots. At the end of a row the consumer stores the row's bf16 value
// for the caller and, tagged, for the stages that read it. A consumer visits only the stages where it owns rows.
template <int KIND>
struct Consumer {
  int s;
  int r, r1, row0;    // current row, end of this consumer's rows, the workgroup's first row of the stage
  int c, C;
  int n, seen;        // chunks consumed; chunks known to have landed
  float acc;
  bool failed;
  uint32_t tag;
  BP_GLOBAL uint16_t* y;   // the stage's outputs
  uint32_t* ty;            // the stage's tagged outputs

  // Moves to stage `from` or the next one with rows for this consumer and waits (bounded) for its input in LDS.
  __device__ __forceinline__ void enter(StageTable st, SetLds& L, int S, int who, int from, uint32_t* tagged) {
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
    y = (BP_GLOBAL uint16_t*)(st[s].y);
    ty = tagged + L.tag_off[s];
    uint32_t it = 0;
    while (!failed && lds_load_relaxed(&L.xready) <= s) {
      if (++it > kSpinCapLds) {
        failed = true;
        record_error(tagged - kWordsHeader);
      }
      __builtin_amdgcn_s_sleep(1);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  }

  // GS chunks of the current row. RESIDENT: the row is exactly these GS chunks and xr holds the stage's input
  // chunks (loaded once per stage), so only the weights are read from LDS.
  template <int GS, bool RESIDENT>
  __device__ __forceinline__ void group(StageTable st, SetLds& L, int S, int who, int lane, uint32_t* tagged,
                                        uint32_t (&xr)[4][Layout<KIND>::kXDwords]) {
    using Lay = Layout<KIND>;
    uint32_t it = 0;
    while (seen < n + GS && !failed) {
      seen = uniform(lds_load_relaxed(&L.landed[who]));
      if (seen >= n + GS) break;
      if (++it > kSpinCapLds) {
        failed = true;
        record_error(tagged - kWordsHeader);
      }
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
    if (lane == 0) lds_store_relaxed(&L.consumed[who], n);
    c += GS;
    if (c == C) {
      const float tot = wave_sum_dpp(acc);
      if (lane == 0) {
        float v = tot;
        if constexpr (KIND == kInt8) v *= L.scale[s & 1][r - row0];
        const uint32_t bits = float_to_bf16_bits(v);
        y[r] = static_cast<uint16_t>(bits);
        st_agent(&ty[r], (tag << 16) | bits);
      }
      acc = 0.f;
      c = 0;
      if (++r == r1) {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane == 0) __hip_atomic_fetch_add(&L.done[s], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        enter(st, L, S, who, s + 1, tagged);
      }
    }
  }

  // R <= 4 rows of two chunks each (C == 2, the input chunks resident in xr): one wait and one round of ring reads
  // for all R rows, their dot chains interleaved, one wave reduction for the four (wave_sum4_rows) and one store
  // instruction per output array (lanes 0, 16, 32, 48 hold the four totals). Short rows (an int8 row of 2048 is
  // 2 KiB) make the per-row wait, reduction and stores the consumer's bound; this divides them by R. Every row of
  // such a stage goes through here (R = 4, then 2 and 1 for the last rows), so its sum order does not depend on
  // where the row falls in a group.
  template <int R>
  __device__ __forceinline__ void rows(StageTable st, SetLds& L, int S, int who, int lane, uint32_t* tagged,
                                       uint32_t (&xr)[4][Layout<KIND>::kXDwords]) {
    constexpr int G = 2 * R;  // chunks
    static_assert(G <= kSetSlots, "the ring holds a consumer's largest group");
    uint32_t it = 0;
    while (seen < n + G && !failed) {
      seen = uniform(lds_load_relaxed(&L.landed[who]));
      if (seen >= n + G) break;
      if (++it > kSpinCapLds) {
        failed = true;
        record_error(tagged - kWordsHeader);
      }
      __builtin_amdgcn_s_sleep(0);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    u32x4 w[G];
    const int slot0 = n % kSetSlots;
    if (slot0 + G <= kSetSlots) {  // the group's slots are contiguous: one address, immediate offsets
      const uint8_t* base = &L.ring[who][slot0][lane * 16];
#pragma unroll
      for (int j = 0; j < G; ++j) w[j] = *reinterpret_cast<const u32x4*>(base + j * 1024);
    } else {
      int slot = slot0;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        w[j] = *reinterpret_cast<const u32x4*>(&L.ring[who][slot][lane * 16]);
        slot = slot + 1 == kSetSlots ? 0 : slot + 1;
      }
    }
    float a[R];
#pragma unroll
    for (int q = 0; q < R; ++q) a[q] = chunk_dot<KIND>(w[2 * q], xr[0], 0.f);
#pragma unroll
    for (int q = 0; q < R; ++q) a[q] = chunk_dot<KIND>(w[2 * q + 1], xr[1], a[q]);
    n += G;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane == 0) lds_store_relaxed(&L.consumed[who], n);
    const float tot = wave_sum4_rows(a[0], a[R > 1 ? 1 : 0], a[R > 2 ? 2 : 0], a[R > 3 ? 3 : 0]);
    const int q = ((lane >> 5) & 1) | ((lane >> 3) & 2);  // row of the total in lanes 0, 16, 32, 48
    if ((lane & 15) == 0 && q < R) {
      float v = tot;
      if constexpr (KIND == kInt8) v *= L.scale[s & 1][r + q - row0];
      const uint32_t bits = float_to_bf16_bits(v);
      y[r + q] = static_cast<uint16_t>(bits);
      st_agent(&ty[r + q], (tag << 16) | bits);
    }
    r += R;
    if (r == r1) {
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if (lane == 0) __hip_atomic_fetch_add(&L.done[s], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      enter(st, L, S, who, s + 1, tagged);
    }
  }

  __device__ __forceinline__ void run(StageTable st, SetLds& L, int S, int who, int lane, uint32_t* tagged) {
    using Lay = Layout<KIND>;
    uint32_t xr[4][Lay::kXDwords];
    enter(st, L, S, who, 0, tagged);
    while (s < S) {
      if (C == 4 || C == 2) {  // one group per row: the stage's input chunks stay in registers
        const int stage = s;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (j < C) {
            const u32x4* xs = reinterpret_cast<const u32x4*>(&L.x[s & 1][j * Lay::kChunk + lane * Lay::kEpl]);
#pragma unroll
            for (int q = 0; q < Lay::kXDwords / 4; ++q) {
              const u32x4 t = xs[q];
              xr[j][4 * q + 0] = t.x;
              xr[j][4 * q + 1] = t.y;
              xr[j][4 * q + 2] = t.z;
              xr[j][4 * q + 3] = t.w;
            }
          }
        }
        if (C == 4) {
          while (s == stage) group<4, true>(st, L, S, who, lane, tagged, xr);
        } else {
          while (s == stage) {
            if (r1 - r >= 4)
              rows<4>(st, L, S, who, lane, tagged, xr);
            else if (r1 - r >= 2)
              rows<2>(st, L, S, who, lane, tagged, xr);
            else
              rows<1>(st, L, S, who, lane, tagged, xr);
          }
        }
      } else if ((C & 3) == 0) {
        group<4, false>(st, L, S, who, lane, tagged, xr);
      } else if ((C & 1) == 0) {
        group<2, false>(st, L, S, who, lane, tagged, xr);
      } else {
        group<1, false>(st, L, S, who, lane, tagged, xr);
      }
    }
  }
};

// Waits (bounded) until `active` consumers of this workgroup are done with stage `stage`.
__device__ __forceinline__ void wait_done(SetLds& L, int stage, int active, bool& failed, uint32_t* scratch) {
  uint32_t it = 0;
  while (!failed && lds_load_relaxed(&L.done[stage]) < active) {
    if (++it > kSpinCapLds) {
      failed = true;
      record_error(scratch);
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

__device__ __forceinline__ int active_consumers(const SetLds& L, int s) {
  int a = 0;
#pragma unroll
  for (int i = 0; i < kSetCW; ++i) a += L.rows[s][i] < L.rows[s][i + 1] ? 1 : 0;
  return a;
}

constexpr int kSetChMax = kSetKMax / 512;  // 512-element chunks of the longest input
constexpr int kSetRound = kSetTin / 512;   // chunks of tagged words gathered per round

// This lane's 8 values of chunk c of the input (4 packed bf16 pairs) and their sum of squares (in element order).
__device__ __forceinline__ float chunk_ss(const uint32_t (&d)[4]) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = bf16_bits_to_float(d[e] & 0xffffu), hi = bf16_bits_to_float(d[e] >> 16);
    ss += lo * lo;
    ss += hi * hi;
  }
  return ss;
}

// Writes the input held in registers (v: each lane's 8 values of every chunk) to xl, renormalised to unit RMS when
// `norm`: mean square = (sum over lanes of the lane's chunk sums of squares, in chunk order) / K,
// x = bf16(x * (1 / sqrt(mean square))); an all-zero vector is left as it is.
__device__ __forceinline__ void write_input(uint32_t (&v)[kSetChMax][4], int K, bool norm, uint16_t* xl,
                                            int lane) {
  const int nch = K / 512;
  float inv = 1.f;
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < kSetChMax; ++c)
      if (c < nch) ss += chunk_ss(v[c]);
    const float ms = wave_sum_dpp(ss) / static_cast<float>(K);
    if (ms > 0.f) inv = 1.f / sqrtf(ms);
  }
#pragma unroll
  for (int c = 0; c < kSetChMax; ++c) {
    if (c < nch) {
      uint32_t d[4] = {v[c][0], v[c][1], v[c][2], v[c][3]};
      if (norm) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = float_to_bf16_bits(bf16_bits_to_float(d[e] & 0xffffu) * inv);
          const uint32_t hi = float_to_bf16_bits(bf16_bits_to_float(d[e] >> 16) * inv);
          d[e] = lo | (hi << 16);
        }
      }
      *reinterpret_cast<u32x4*>(xl + c * 512 + lane * 8) = u32x4{d[0], d[1], d[2], d[3]};
    }
  }
}

// Reads round H of the K published rows at rows_t (tagged words) into registers: chunks H * kSetRound ..
// (up to kSetRound chunks of 512 words, LDS-DMA into the staging buffer, device scope). A chunk is read again until
// all of its words carry `tag` (bounded), then unpacked two words at a time (their tags into one dword, their
// values into another).
template <int H>
__device__ __forceinline__ void gather_round(const uint32_t* __restrict__ rows_t, int K, uint32_t tag, SetLds& L,
                                             uint32_t (&v)[kSetChMax][4], int lane,
                                             bool& failed, uint32_t* scratch) {
  const int hn = min(kSetRound, K / 512 - H * kSetRound);
  const uint32_t tag2 = tag | (tag << 16);
  uint32_t pending = (1u << hn) - 1u;  // wave-uniform
  uint32_t it = 0;
  while (true) {
#pragma unroll
    for (int c = 0; c < kSetRound; ++c) {
      if (!((pending >> c) & 1u)) continue;
#pragma unroll
      for (int q = 0; q < 2; ++q)
        __builtin_amdgcn_global_load_lds((const BP_GLOBAL void*)(rows_t + (H * kSetRound + c) * 512 + q * 256 + lane * 4),
                                         (BP_LDS void*)&L.tin[c * 512 + q * 256], 16, 0, kDeviceScope);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm<0>());
#pragma unroll
    for (int c = 0; c < kSetRound; ++c) {
      if (!((pending >> c) & 1u)) continue;
      const u32x4* tp = reinterpret_cast<const u32x4*>(&L.tin[c * 512 + lane * 8]);
      const u32x4 a = tp[0], b = tp[1];
      const uint32_t t0 = (a.y & 0xffff0000u) | (a.x >> 16), t1 = (a.w & 0xffff0000u) | (a.z >> 16);
      const uint32_t t2 = (b.y & 0xffff0000u) | (b.x >> 16), t3 = (b.w & 0xffff0000u) | (b.z >> 16);
      const bool ok = t0 == tag2 && t1 == tag2 && t2 == tag2 && t3 == tag2;
      if (__all(ok) || failed) {
        uint32_t(&d)[4] = v[H * kSetRound + c];
        d[0] = (a.y << 16) | (a.x & 0xffffu);
        d[1] = (a.w << 16) | (a.z & 0xffffu);
        d[2] = (b.y << 16) | (b.x & 0xffffu);
        d[3] = (b.w << 16) | (b.z & 0xffffu);
        pending &= ~(1u << c);
      }
    }
    if (pending == 0u) break;
    if (++it > kSpinCapGlobal && !failed) {
      failed = true;
      record_error(scratch);
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

static_assert(kSetChMax == 2 * kSetRound, "the input is gathered in two rounds");

// Reads an external input vector (K bf16 at src) into registers.
__device__ __forceinline__ void load_input(const BP_GLOBAL uint16_t* src, int K, uint32_t (&v)[kSetChMax][4],
                                           int lane) {
  const int nch = K / 512;
#pragma unroll
  for (int c = 0; c < kSetChMax; ++c) {
    if (c < nch) {
      const u32x4 t = *reinterpret_cast<GlobalVec>(src + c * 512 + lane * 8);
      v[c][0] = t.x;
      v[c][1] = t.y;
      v[c][2] = t.z;
      v[c][3] = t.w;
    }
  }
}

// The workgroup's sync wave: the input of every stage into LDS, in stage order.
template <int KIND>
__device__ __forceinline__ void sync_wave(StageTable st, int S, uint32_t* __restrict__ scratch, SetLds& L,
                                          int scale_dt, int lane) {
  const int g = blockIdx.x;
  uint32_t* tagged = scratch + kWordsHeader;
  const uint32_t tag = L.tag;
  bool failed = false;

  for (int s = 0; s < S; ++s) {
    const int K = st[s].K;
    const int nch = K / 512;
    uint16_t* xl = L.x[s & 1];
    const int ws = st[s].wait_stage;

    // Loads that depend on no other stage go out first, so that their latency (a few us behind the weight stream)
    // overlaps the wait for this stage's LDS buffers: an external input vector, and the int8 row scales of the
    // stage (the consumers apply them at the ends of their rows).
    uint32_t v[kSetChMax][4];
    if (ws < 0) load_input((const BP_GLOBAL uint16_t*)(st[s].src), K, v, lane);
    float sc[kSetRowsMax / kWave];
    int rows = 0;
    if constexpr (KIND == kInt8) {
      const int row0 = L.rows[s][0];
      rows = L.rows[s][kSetCW] - row0;
#pragma unroll
      for (int j = 0; j < kSetRowsMax / kWave; ++j) {
        const int i = lane + j * kWave;
        if (i < rows) {
          const int row = row0 + i;
          int seg = 0, seg_begin = 0;
          while (st[s].seg_end[seg] <= row) seg_begin = st[s].seg_end[seg++];
          sc[j] = load_scale(st[s].scale[seg], row - seg_begin, scale_dt);
        }
      }
    }

    // x[s & 1] and scale[s & 1] were last used by stage s - 2
    if (s >= 2) wait_done(L, s - 2, active_consumers(L, s - 2), failed, scratch);
    if constexpr (KIND == kInt8) {
#pragma unroll
      for (int j = 0; j < kSetRowsMax / kWave; ++j)
        if (lane + j * kWave < rows) L.scale[s & 1][lane + j * kWave] = sc[j];
    }

    // the input vector: published rows of an earlier stage (read once this workgroup's own consumers are done
    // with that stage: the other workgroups finish it at about the same time), or the external vector loaded above
    if (ws >= 0) {
      wait_done(L, ws, active_consumers(L, ws), failed, scratch);
      const int64_t e0 = (static_cast<const char*>(st[s].src) - static_cast<const char*>(st[ws].y)) / 2;
      gather_round<0>(tagged + L.tag_off[ws] + e0, K, tag, L, v, lane, failed, scratch);
      if (K > kSetRound * 512) gather_round<1>(tagged + L.tag_off[ws] + e0, K, tag, L, v, lane, failed, scratch);
    }
    write_input(v, K, st[s].renorm != 0, xl, lane);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane == 0) lds_store_relaxed(&L.xready, s + 1);
    // the input as used, for the caller (x[s & 1] stays unchanged until stage s + 2)
    if (g == 0 && st[s].x_used != nullptr) {
      BP_GLOBAL uint16_t* xu = (BP_GLOBAL uint16_t*)(st[s].x_used);
      for (int c0 = 0; c0 < nch; ++c0)
        *reinterpret_cast<BP_GLOBAL u32x4*>(xu + c0 * 512 + lane * 8) =
            *reinterpret_cast<const u32x4*>(xl + c0 * 512 + lane * 8);
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
  for (int s = threadIdx.x; s < S; s += kSetThreads) lds.done[s] = 0;
  if (threadIdx.x < kSetCW) {
    lds.landed[threadIdx.x] = 0;
    lds.consumed[threadIdx.x] = 0;
  }
  if (threadIdx.x == 0) {
    int32_t off = 0;
    for (int s = 0; s < S; ++s) {
      lds.tag_off[s] = off;
      off += (st[s].N + 7) & ~7;
    }
    lds.xready = 0;
    // launch generation: every workgroup of the previous launches added 1 to the launch counter
    const uint32_t gen = ld_agent(&scratch[0]) / gridDim.x;
    lds.tag = gen % 65535u + 1u;  // 1..65535: a zeroed scratch holds no valid row
  }
  __syncthreads();
  if (wave == kSetSyncWave) {
    sync_wave<KIND>(st, S, scratch, lds, scale_dt, lane);
  } else if (wave >= kSetCW) {
    // Issue priority over the consumer sharing its SIMD: the producer issues a few instructions per chunk and must
    // keep the weight loads flowing; at equal priority a VALU-heavy consumer (int8 conversion) delays them.
    __builtin_amdgcn_s_setprio(3);
    producer_wave<KIND>(st, lds, S, wave - kSetCW, lane, scratch);
  } else {
    Consumer<KIND> cons;
    cons.failed = false;
    cons.n = 0;
    cons.seen = 0;
    cons.tag = lds.tag;
    cons.run(st, lds, S, wave, lane, scratch + kWordsHeader);
  }
}

int set_validate(const BpSetStage* st, int S, int wkind, int G) {
  if (st == nullptr || S <= 0 || G <= 0) return BP_E_INVALID_ARG;
  if (S > kSetStagesMax) return BP_E_UNSUPPORTED;
  if (wkind != kBf16 && wkind != kInt8) return BP_E_UNSUPPORTED;
  if (G > 65536) return BP_E_UNSUPPORTED;
  const int64_t chunk = wkind == kBf16 ? 512 : 1024;
  int64_t words = 0;
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

int64_t scratch_words(const BpSetStage* st, int S) {
  int64_t words = kWordsHeader;
  for (int s = 0; s < S; ++s) words += (st[s].N + 7) & ~7;
  return words;
}

}  // namespace
}  // namespace bp

extern "C" {

size_t bp_linear_set_scratch_bytes(const BpSetStage* stages, int num_stages, int num_workgroups) {
  if (stages == nullptr || num_stages <= 0 || num_workgroups <= 0) return 0;
  return static_cast<size_t>(bp::scratch_words(stages, num_stages)) * sizeof(uint32_t);
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
