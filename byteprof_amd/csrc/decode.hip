// The non-linear steps of one OLMo-2 decode step (batch 1, one new token), for a decode loop whose every launch
// lives in one captured HIP graph: the token id and the position are read from device memory, and the last step
// writes the next token and advances the position, so a replay needs no host value.
//
//   embed           x <- table[tok]
//   qk_rope_cache   q, k <- RMSNorm over the whole projection (fp32, weight applied in fp32, rounded to bf16),
//                   rotated by RoPE at pos (cos / sin in fp32, one rounding), k and v written to the cache at pos
//   rope_attention  qk_rope_cache and attention fused, one workgroup per head (the decode loop's path)
//   attention       per head: s_t = bf16(bf16(q . k_t) * scale) for t <= pos, p = bf16(softmax_fp32(s)),
//                   out = bf16(sum_t p_t v_t)
//   norm_residual   out <- bf16(residual + bf16(w * x * rsqrt(mean(x^2) + eps))) (no residual: the plain norm;
//                   the mean square in wave_sumsq's order, common.h)
//   silu_mul        out <- bf16(bf16(silu(g)) * u), g and u the two halves of the fused gate|up projection
//   argmax_next     tok <- first index of the largest logit (NaN counts as largest); pos <- pos + 1
//
// The roundings are those of transformers' Olmo2ForCausalLM run in bf16 with the eager attention, the model whose
// forward the reference's decode loop replays (byteprof/optim/olmo.py:122-219: make_generate_graph captures the
// forward, the argmax and the next-step input updates in one graph).

#include <climits>

#include "byteprof_amd.h"
#include "common.h"

namespace bp {
namespace {

constexpr int kBlock = 1024;       // threads of the one-workgroup kernels
constexpr int kAttnThreads = 512;  // threads per head in the attention
constexpr int kAttnMaxLen = 4096;  // positions a cache may hold (scores in LDS)

// Sum of v over the workgroup (blockDim.x a multiple of 64, at most kBlock); every thread gets the total.
__device__ float block_sum(float v, float* red) {
  v = xor_butterfly<true>(v, AddOp{});
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, waves = blockDim.x / kWave;
  __syncthreads();  // red may still be read by a previous call
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < waves; ++i) t += red[i];
  return t;
}

__device__ float block_max(float v, float* red) {
  v = xor_butterfly<true>(v, MaxOp{});
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, waves = blockDim.x / kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
  for (int i = 1; i < waves; ++i) t = fmaxf(t, red[i]);
  return t;
}

__device__ __forceinline__ float ld_bf16(const uint16_t* p, int64_t i) { return bf16_bits_to_float(p[i]); }

// grid = rows: x[r] <- table[tok[r]].
__global__ __launch_bounds__(kBlock) void embed_kernel(const int64_t* __restrict__ tok,
                                                       const uint16_t* __restrict__ table,
                                                       uint16_t* __restrict__ x, int H, int64_t V) {
  int64_t t = tok[blockIdx.x];
  t = t < 0 ? 0 : (t >= V ? V - 1 : t);  // ids are validated on the host; the clamp keeps the read in bounds
  uint16_t* xr = x + static_cast<int64_t>(blockIdx.x) * H;
  for (int i = threadIdx.x; i < H; i += blockDim.x) xr[i] = table[t * H + i];
}


constexpr int kAttnUnroll = 4;  // row batches whose loads are in flight together

// q_row . w_row for 8 bf16 cache values packed in w and 8 q values: the products summed in order.
__device__ __forceinline__ float dot8(const u32x4& w, const float (&qv)[8]) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
  float dot = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    dot += bf16_bits_to_float(wd[e] & 0xffffu) * qv[2 * e];
    dot += bf16_bits_to_float(wd[e] >> 16) * qv[2 * e + 1];
  }
  return dot;
}

// Sum of v over each group of LPR consecutive lanes (LPR a power of two <= 32), returned to every lane of the
// group: DPP pairs within quads, quads within half-rows, half-rows within rows of 16, then rows of 16 in pairs.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (LPR >= 2) v += dpp_f32<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  if constexpr (LPR >= 4) v += dpp_f32<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  if constexpr (LPR >= 8) v += dpp_f32<0x141, 0xF>(v);  // row_half_mirror
  if constexpr (LPR >= 16) v += dpp_f32<0x140, 0xF>(v); // row_mirror
  if constexpr (LPR >= 32) v = xor_stage<16>(v, AddOp{});
  return v;
}

// Sum (or maximum) of v over the wave, returned to every lane (an xor butterfly, distances 32 .. 1).
__device__ __forceinline__ float wave_sum(float v) { return xor_butterfly<true>(v, AddOp{}); }
__device__ __forceinline__ float wave_max(float v) { return xor_butterfly<true>(v, MaxOp{}); }

constexpr int kAttnWaves = kAttnThreads / kWave;

// One head's attention over its cache rows K, V ([max_len, D] bf16, 16-byte aligned, D = 8 * LPR) at positions
// 0 .. T-1, run by the workgroup's kAttnThreads threads. Layout: LPR lanes per cache row (16 bytes each), 64 / LPR
// rows per wave instruction, the waves on consecutive rows, and kAttnUnroll such row batches loaded before they
// are used. The first batch of K and V rows can be loaded early (prefetch(), before the caller's own work), so that
// its latency overlaps the caller's; a row can be taken from LDS instead of the cache (SUB: the row the caller
// writes in this launch). Scores: a lane's 8 products in order, then the row's lanes summed (group_sum);
// s_t = bf16(bf16(q . k_t) * scale), p = bf16(softmax_fp32(s)). Values: each lane accumulates its 8 dimensions
// over its rows; the row groups of a wave are added by lane butterflies, the waves' sums in wave order through LDS.
template <int LPR, bool SUB>
struct HeadAttention {
  static constexpr int D = 8 * LPR;
  static constexpr int RPW = kWave / LPR;           // rows per wave instruction
  static constexpr int STEP = kAttnWaves * RPW;     // rows per workgroup-wide batch
  static constexpr int BATCH = kAttnUnroll * STEP;  // rows per round of loads
  // the rows 0 .. T-1 of K and V as buffer resources: a row at or past T has an offset past its resource, so its
  // load returns zeros without a memory request (and without a branch around the load)
  __amdgpu_buffer_rsrc_t krs, vrs;
  int T, s, slot;
  u32x4 k0[kAttnUnroll], v0[kAttnUnroll];

  __device__ __forceinline__ HeadAttention(const uint16_t* K_, const uint16_t* V_, int T_)
      : krs(buffer_rsrc(K_, 2 * T_ * D)), vrs(buffer_rsrc(V_, 2 * T_ * D)), T(T_) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    s = lane % LPR;
    slot = wave * RPW + lane / LPR;  // this lane's row within a batch
  }

  __device__ __forceinline__ void load_batch(__amdgpu_buffer_rsrc_t rs, int t0, u32x4 (&out)[kAttnUnroll]) const {
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
      const int t = t0 + u * STEP + slot;
      const uint32_t off = t < T ? static_cast<uint32_t>(2 * (t * D + 8 * s)) : 0x80000000u;
      out[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
  }

  // Issues the loads of the first batch of K and V rows.
  __device__ __forceinline__ void prefetch() {
    load_batch(krs, 0, k0);
    load_batch(vrs, 0, v0);
  }

  __device__ __forceinline__ void scores(const u32x4 (&kv)[kAttnUnroll], int t0, const float (&qv)[8],
                                         const uint16_t* ksub, int sub_lo, float scale, float* sc, float& m) const {
    float dot[kAttnUnroll];
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
      const int t = t0 + u * STEP + slot;
      const u32x4 w = SUB && t >= sub_lo && t < T ? *reinterpret_cast<const u32x4*>(ksub + (t - sub_lo) * D + 8 * s)
                                                  : kv[u];
      dot[u] = dot8(w, qv);
    }
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) dot[u] = group_sum<LPR>(dot[u]);
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
      const int t = t0 + u * STEP + slot;
      if (t < T) {
        const float v = round_to_bf16(round_to_bf16(dot[u]) * scale);
        if (s == 0) sc[t] = v;
        m = fmaxf(m, v);
      }
    }
  }

  __device__ __forceinline__ void values(const u32x4 (&vv)[kAttnUnroll], int t0, const uint16_t* vsub, int sub_lo,
                                         const float* sc, float inv, float (&acc)[8]) const {
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
      const int t = t0 + u * STEP + slot;
      if (t < T) {
        const u32x4 w = SUB && t >= sub_lo ? *reinterpret_cast<const u32x4*>(vsub + (t - sub_lo) * D + 8 * s) : vv[u];
        const float p = round_to_bf16(sc[t] * inv);
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[2 * e] += p * bf16_bits_to_float(wd[e] & 0xffffu);
          acc[2 * e + 1] += p * bf16_bits_to_float(wd[e] >> 16);
        }
      }
    }
  }

  // q: bf16 values in LDS qs[0 .. D). Rows t >= sub_lo (INT_MAX: none) are read from ksub / vsub [t - sub_lo][D]
  // (bf16, LDS, 16-byte aligned rows) instead of the cache. Writes out[0 .. D). The caller has made qs, ksub and
  // vsub visible (a barrier).
  // LDS: sc[T] scores, red_m / red_l [kAttnWaves], part [kAttnWaves * D].
  __device__ __forceinline__ void run(const float* qs, const uint16_t* ksub, const uint16_t* vsub, int sub_lo,
                                      float scale, float* sc, float* red_m, float* red_l, float* part,
                                      uint16_t* __restrict__ out) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    float qv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[e] = qs[8 * s + e];
    float m = -INFINITY;
    scores(k0, 0, qv, ksub, sub_lo, scale, sc, m);
    for (int t0 = BATCH; t0 < T; t0 += BATCH) {
      u32x4 kv[kAttnUnroll];
      load_batch(krs, t0, kv);
      scores(kv, t0, qv, ksub, sub_lo, scale, sc, m);
    }
    m = wave_max(m);
    if (lane == 0) red_m[wave] = m;
    __syncthreads();  // also orders the sc writes before the reads below
    m = red_m[0];
    for (int w = 1; w < kAttnWaves; ++w) m = fmaxf(m, red_m[w]);
    float l = 0.f;
    for (int t = threadIdx.x; t < T; t += kAttnThreads) {
      const float e = expf(sc[t] - m);
      sc[t] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) red_l[wave] = l;
    __syncthreads();  // also orders the sc writes before the reads below
    l = red_l[0];
    for (int w = 1; w < kAttnWaves; ++w) l += red_l[w];
    const float inv = 1.f / l;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
    values(v0, 0, vsub, sub_lo, sc, inv, acc);
    for (int t0 = BATCH; t0 < T; t0 += BATCH) {
      u32x4 vv[kAttnUnroll];
      load_batch(vrs, t0, vv);
      values(vv, t0, vsub, sub_lo, sc, inv, acc);
    }
    // the wave's row groups (lanes s, s + LPR, s + 2 LPR, ...) added by butterflies over the group bits
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = xor_butterfly<false, LPR>(acc[e], AddOp{});
    if (lane < LPR) {
#pragma unroll
      for (int e = 0; e < 8; ++e) part[wave * D + 8 * s + e] = acc[e];
    }
    __syncthreads();
    for (int d = threadIdx.x; d < D; d += kAttnThreads) {
      float t = part[d];
      for (int w = 1; w < kAttnWaves; ++w) t += part[w * D + d];
      out[d] = float_to_bf16_bits(t);
    }
  }
};

constexpr int kAttnPart = kAttnWaves * 256;  // floats of the value partials: waves x D (D <= 256)

// 1 / rms of q[0 .. H) and of k[0 .. H) (+ eps inside the root), by a kAttnThreads-thread workgroup: thread t sums
// the squares of elements 8t .. 8t + 7 (then + 8 * kAttnThreads ...) in order, each wave by a butterfly, the waves in
// order. Both attention paths use it, so their q and k are equal bit for bit.
__device__ __forceinline__ void qk_rms(const uint16_t* q, const uint16_t* k, int H, float eps, float* red_q,
                                       float* red_k, float& rq, float& rk) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  float sq = 0.f, sk = 0.f;
  for (int i = 8 * threadIdx.x; i < H; i += 8 * kAttnThreads) {
    const u32x4 qa = *reinterpret_cast<const u32x4*>(q + i);
    const u32x4 ka = *reinterpret_cast<const u32x4*>(k + i);
    const uint32_t qd[4] = {qa.x, qa.y, qa.z, qa.w}, kd[4] = {ka.x, ka.y, ka.z, ka.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float q0 = bf16_bits_to_float(qd[e] & 0xffffu), q1 = bf16_bits_to_float(qd[e] >> 16);
      const float k0 = bf16_bits_to_float(kd[e] & 0xffffu), k1 = bf16_bits_to_float(kd[e] >> 16);
      sq += q0 * q0;
      sq += q1 * q1;
      sk += k0 * k0;
      sk += k1 * k1;
    }
  }
  sq = wave_sum(sq);
  sk = wave_sum(sk);
  if (lane == 0) {
    red_q[wave] = sq;
    red_k[wave] = sk;
  }
  __syncthreads();
  sq = red_q[0];
  sk = red_k[0];
  for (int w = 1; w < kAttnWaves; ++w) {
    sq += red_q[w];
    sk += red_k[w];
  }
  rq = 1.f / sqrtf(sq / static_cast<float>(H) + eps);
  rk = 1.f / sqrtf(sk / static_cast<float>(H) + eps);
}

// The RoPE pair (a, a + D/2) of head h at position pos: q and k normalised (weights in fp32, bf16 rounding), rotated
// with fp32 cos / sin; returns the rotated q as bf16 values and k as bf16 bits.
struct RopePair {
  float qa, qb;
  uint16_t ka, kb;
};
__device__ __forceinline__ RopePair rope_pair(float fqa, float fqb, float fka, float fkb, float wqa, float wqb,
                                              float wka, float wkb, float fr, int64_t pos, float rq, float rk) {
  const float f = fr * static_cast<float>(pos);
  const float c = cosf(f), sn = sinf(f);
  const float qa = round_to_bf16(wqa * (fqa * rq));
  const float qb = round_to_bf16(wqb * (fqb * rq));
  const float ka = round_to_bf16(wka * (fka * rk));
  const float kb = round_to_bf16(wkb * (fkb * rk));
  RopePair r;
  r.qa = round_to_bf16(qa * c + (-qb) * sn);
  r.qb = round_to_bf16(qb * c + qa * sn);
  r.ka = float_to_bf16_bits(ka * c + (-kb) * sn);
  r.kb = float_to_bf16_bits(kb * c + ka * sn);
  return r;
}

// grid = rows: row r of qkv [rows, 3H] at position *pos_p + r: q, k normalised over the whole projection (qk_rms)
// and rotated (rope_pair) for every head; q -> q_out[r]; k, v -> the caches at that position (if inside them).
__global__ __launch_bounds__(kAttnThreads) void qk_rope_cache_kernel(const uint16_t* __restrict__ qkv,
                                                                     const uint16_t* __restrict__ qw,
                                                                     const uint16_t* __restrict__ kw,
                                                                     const float* __restrict__ inv_freq,
                                                                     const int64_t* __restrict__ pos_p,
                                                                     uint16_t* __restrict__ q_out,
                                                                     uint16_t* __restrict__ kc,
                                                                     uint16_t* __restrict__ vc, int heads, int D,
                                                                     int max_len, float eps) {
  __shared__ float red_q[kAttnWaves], red_k[kAttnWaves];
  const int r = blockIdx.x;
  const int H = heads * D, half = D / 2;
  const int64_t pos = *pos_p + r;
  const bool in_cache = pos >= 0 && pos < max_len;
  const uint16_t* q = qkv + static_cast<int64_t>(r) * 3 * H;
  const uint16_t* k = q + H;
  const uint16_t* v = q + 2 * H;
  uint16_t* qo = q_out + static_cast<int64_t>(r) * H;
  float rq, rk;
  qk_rms(q, k, H, eps, red_q, red_k, rq, rk);
  for (int i = threadIdx.x; i < H / 2; i += kAttnThreads) {
    const int h = i / half, j = i % half;
    const int a = h * D + j, b = a + half;
    const RopePair rp = rope_pair(ld_bf16(q, a), ld_bf16(q, b), ld_bf16(k, a), ld_bf16(k, b), ld_bf16(qw, a),
                                  ld_bf16(qw, b), ld_bf16(kw, a), ld_bf16(kw, b), inv_freq[j], pos, rq, rk);
    qo[a] = float_to_bf16_bits(rp.qa);
    qo[b] = float_to_bf16_bits(rp.qb);
    if (in_cache) {
      const int64_t row = (static_cast<int64_t>(h) * max_len + pos) * D;
      kc[row + j] = rp.ka;
      kc[row + j + half] = rp.kb;
      vc[row + j] = v[a];
      vc[row + j + half] = v[b];
    }
  }
}

// grid = (heads, rows); row r of q / out [rows, heads * D] attends over positions 0 .. *pos_p + r of the head's
// cache rows [max_len, D], D = 8 * LPR.
template <int LPR>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(const uint16_t* __restrict__ q,
                                                                 const uint16_t* __restrict__ kc,
                                                                 const uint16_t* __restrict__ vc,
                                                                 const int64_t* __restrict__ pos_p,
                                                                 uint16_t* __restrict__ out, int max_len,
                                                                 float scale) {
  constexpr int D = 8 * LPR;
  __shared__ float sc[kAttnMaxLen];
  __shared__ float qs[D];
  __shared__ float red_m[kAttnWaves], red_l[kAttnWaves];
  __shared__ float part[kAttnPart];
  const int h = blockIdx.x, r = blockIdx.y;
  const int64_t row = (static_cast<int64_t>(r) * gridDim.x + h) * D;
  int64_t pos = *pos_p + r;
  pos = pos < 0 ? 0 : (pos >= max_len ? max_len - 1 : pos);
  HeadAttention<LPR, false> att(kc + static_cast<int64_t>(h) * max_len * D,
                                vc + static_cast<int64_t>(h) * max_len * D, static_cast<int>(pos) + 1);
  att.prefetch();
  for (int d = threadIdx.x; d < D; d += kAttnThreads) qs[d] = ld_bf16(q, row + d);
  __syncthreads();
  att.run(qs, nullptr, nullptr, INT_MAX, scale, sc, red_m, red_l, part, out + row);
}

// qk_rope_cache and attention in one launch: every workgroup h computes the q / k norms over the whole projections
// (the same sums in every workgroup, in qk_rope_cache_kernel's order: the results are equal bit for bit to the two
// launches), rotates its own head, writes its k and v at pos to the cache, and attends over positions
// 0 .. pos with that row taken from LDS. Every load that does not depend on the norms (the projections, the RoPE
// operands, the first batch of cache rows) is issued before the first reduction.
template <int LPR>
__global__ __launch_bounds__(kAttnThreads) void rope_attention_kernel(const uint16_t* __restrict__ qkv,
                                                                      const uint16_t* __restrict__ qw,
                                                                      const uint16_t* __restrict__ kw,
                                                                      const float* __restrict__ inv_freq,
                                                                      const int64_t* __restrict__ pos_p,
                                                                      uint16_t* __restrict__ kc,
                                                                      uint16_t* __restrict__ vc,
                                                                      uint16_t* __restrict__ out, int heads,
                                                                      int max_len, float eps, float scale) {
  constexpr int D = 8 * LPR;
  constexpr int half = D / 2;
  __shared__ float sc[kAttnMaxLen];
  __shared__ float qs[D];
  __shared__ __align__(16) uint16_t ks[D];
  __shared__ __align__(16) uint16_t vs[D];
  __shared__ float red_q[kAttnWaves], red_k[kAttnWaves], red_m[kAttnWaves], red_l[kAttnWaves];
  __shared__ float part[kAttnPart];
  const int h = blockIdx.x;
  const int H = heads * D;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t pos_in = *pos_p;
  const bool in_cache = pos_in >= 0 && pos_in < max_len;
  const int64_t pos = pos_in < 0 ? 0 : (pos_in >= max_len ? max_len - 1 : pos_in);
  const uint16_t* q = qkv;
  const uint16_t* k = qkv + H;
  const uint16_t* v = qkv + 2 * H;
  uint16_t* K = kc + static_cast<int64_t>(h) * max_len * D;
  uint16_t* V = vc + static_cast<int64_t>(h) * max_len * D;

  // RoPE operands of this thread's pair (j, j + D/2) of head h (threads j < D/2; D <= 256 <= threads)
  const int j = threadIdx.x;
  const bool roper = j < half;
  const int a = h * D + j, b = a + half;
  float f_qa = 0.f, f_qb = 0.f, f_ka = 0.f, f_kb = 0.f, w_qa = 0.f, w_qb = 0.f, w_ka = 0.f, w_kb = 0.f, fr = 0.f;
  uint16_t v_a = 0, v_b = 0;
  if (roper) {
    f_qa = ld_bf16(q, a);
    f_qb = ld_bf16(q, b);
    f_ka = ld_bf16(k, a);
    f_kb = ld_bf16(k, b);
    w_qa = ld_bf16(qw, a);
    w_qb = ld_bf16(qw, b);
    w_ka = ld_bf16(kw, a);
    w_kb = ld_bf16(kw, b);
    v_a = v[a];
    v_b = v[b];
    fr = inv_freq[j];
  }
  HeadAttention<LPR, true> att(K, V, static_cast<int>(pos) + 1);
  att.prefetch();

  // the norms over the whole projections
  float rq, rk;
  qk_rms(q, k, H, eps, red_q, red_k, rq, rk);
  if (roper) {
    const RopePair rp = rope_pair(f_qa, f_qb, f_ka, f_kb, w_qa, w_qb, w_ka, w_kb, fr, pos_in, rq, rk);
    qs[j] = rp.qa;
    qs[j + half] = rp.qb;
    const uint16_t k_lo = rp.ka;
    const uint16_t k_hi = rp.kb;
    ks[j] = k_lo;
    ks[j + half] = k_hi;
    vs[j] = v_a;
    vs[j + half] = v_b;
    if (in_cache) {
      const int64_t r = pos_in * D;
      K[r + j] = k_lo;
      K[r + j + half] = k_hi;
      V[r + j] = v_a;
      V[r + j + half] = v_b;
    }
  }
  __syncthreads();  // qs, ks and vs, written above, are read below
  att.run(qs, ks, vs, in_cache ? static_cast<int>(pos_in) : INT_MAX, scale, sc, red_m, red_l, part,
          out + static_cast<int64_t>(h) * D);
}

constexpr int kRowsMax = 16;  // rows of one fused verify launch

// grid = (heads, rows): workgroup (h, r) attends for row r of qkv [rows, 3H], at position *pos_p + r, over positions
// 0 .. *pos_p + r. The rows 0 .. r of the launch for its own head are normalised (qk_rms's order) and rotated
// (rope_pair) in this workgroup and read from LDS, the positions before them from the cache; the workgroup writes
// only its own row's k and v to the cache. Equal bit for bit to qk_rope_cache_kernel + attention_kernel on the same
// rows (the same sums in the same order).
template <int LPR>
__global__ __launch_bounds__(kAttnThreads) void rope_attention_rows_kernel(const uint16_t* __restrict__ qkv,
                                                                           const uint16_t* __restrict__ qw,
                                                                           const uint16_t* __restrict__ kw,
                                                                           const float* __restrict__ inv_freq,
                                                                           const int64_t* __restrict__ pos_p,
                                                                           uint16_t* __restrict__ kc,
                                                                           uint16_t* __restrict__ vc,
                                                                           uint16_t* __restrict__ out, int heads,
                                                                           int max_len, float eps, float scale) {
  constexpr int D = 8 * LPR;
  constexpr int half = D / 2;
  __shared__ float sc[kAttnMaxLen];
  __shared__ float qs[D];
  __shared__ __align__(16) uint16_t ks[kRowsMax * D];
  __shared__ __align__(16) uint16_t vs[kRowsMax * D];
  __shared__ float red_q[kAttnWaves], red_k[kRowsMax][kAttnWaves], red_m[kAttnWaves], red_l[kAttnWaves];
  __shared__ float part[kAttnPart];
  const int h = blockIdx.x, r = blockIdx.y;
  const int H = heads * D;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t pos0 = *pos_p;
  const int64_t pos_r = pos0 + r;
  const bool in_cache = pos_r >= 0 && pos_r < max_len;
  const int64_t posc = pos_r < 0 ? 0 : (pos_r >= max_len ? max_len - 1 : pos_r);
  uint16_t* K = kc + static_cast<int64_t>(h) * max_len * D;
  uint16_t* V = vc + static_cast<int64_t>(h) * max_len * D;
  HeadAttention<LPR, true> att(K, V, static_cast<int>(posc) + 1);
  att.prefetch();

  // RoPE operands of this thread's (row, pair) items: item i = threadIdx.x + p * kAttnThreads is pair i % (D/2) of
  // row i / (D/2); rows past r load row r (in bounds; not used). All loaded before the first reduction.
  constexpr int kPass = (kRowsMax * half + kAttnThreads - 1) / kAttnThreads;
  const int row3 = 3 * H;
  const int jp = threadIdx.x % half;
  const int a = h * D + jp, b = a + half;
  const float wqa = ld_bf16(qw, a), wqb = ld_bf16(qw, b), wka = ld_bf16(kw, a), wkb = ld_bf16(kw, b);
  const float fr = inv_freq[jp];
  float f_qa[kPass], f_qb[kPass], f_ka[kPass], f_kb[kPass];
  uint16_t v_a[kPass], v_b[kPass];
#pragma unroll
  for (int p = 0; p < kPass; ++p) {
    const int j = (threadIdx.x + p * kAttnThreads) / half;
    const uint16_t* qj = qkv + static_cast<int64_t>(j <= r ? j : r) * row3;
    f_qa[p] = ld_bf16(qj, a);
    f_qb[p] = ld_bf16(qj, b);
    f_ka[p] = ld_bf16(qj + H, a);
    f_kb[p] = ld_bf16(qj + H, b);
    v_a[p] = qj[2 * H + a];
    v_b[p] = qj[2 * H + b];
  }

  // sums of squares of q (row r) and k (rows 0 .. r), each in qk_rms's order; the k rows through a buffer resource
  // over the launch's rows, rows past r at an offset past it (zeros, no memory request; their sums are unused)
  float sq = 0.f;
  float sk[kRowsMax];
#pragma unroll
  for (int j = 0; j < kRowsMax; ++j) sk[j] = 0.f;
  const __amdgpu_buffer_rsrc_t qkv_rs = buffer_rsrc(qkv, 2 * static_cast<int>(gridDim.y) * row3);
  for (int i = 8 * threadIdx.x; i < H; i += 8 * kAttnThreads) {
    u32x4 kx[kRowsMax];
#pragma unroll
    for (int j = 0; j < kRowsMax; ++j) {
      const uint32_t off = j <= r ? static_cast<uint32_t>(2 * (j * row3 + H + i)) : 0x80000000u;
      kx[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qkv_rs, off, 0, 0));
    }
    const u32x4 qa = *reinterpret_cast<const u32x4*>(qkv + static_cast<int64_t>(r) * row3 + i);
    const uint32_t qd[4] = {qa.x, qa.y, qa.z, qa.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float q0 = bf16_bits_to_float(qd[e] & 0xffffu), q1 = bf16_bits_to_float(qd[e] >> 16);
      sq += q0 * q0;
      sq += q1 * q1;
    }
#pragma unroll
    for (int j = 0; j < kRowsMax; ++j) {
      const uint32_t kd[4] = {kx[j].x, kx[j].y, kx[j].z, kx[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float k0 = bf16_bits_to_float(kd[e] & 0xffffu), k1 = bf16_bits_to_float(kd[e] >> 16);
        sk[j] += k0 * k0;
        sk[j] += k1 * k1;
      }
    }
  }
  sq = wave_sum(sq);
  if (lane == 0) red_q[wave] = sq;
#pragma unroll
  for (int j = 0; j < kRowsMax; ++j) {
    if (j <= r) {
      const float t = wave_sum(sk[j]);
      if (lane == 0) red_k[j][wave] = t;
    }
  }
  __syncthreads();
  sq = red_q[0];
  for (int w = 1; w < kAttnWaves; ++w) sq += red_q[w];
  const float rq = 1.f / sqrtf(sq / static_cast<float>(H) + eps);
#pragma unroll
  for (int p = 0; p < kPass; ++p) {
    const int j = (threadIdx.x + p * kAttnThreads) / half;
    if (j <= r) {
      float skj = red_k[j][0];
      for (int w = 1; w < kAttnWaves; ++w) skj += red_k[j][w];
      const float rk = 1.f / sqrtf(skj / static_cast<float>(H) + eps);
      const RopePair rp =
          rope_pair(f_qa[p], f_qb[p], f_ka[p], f_kb[p], wqa, wqb, wka, wkb, fr, pos0 + j, rq, rk);
      ks[j * D + jp] = rp.ka;
      ks[j * D + jp + half] = rp.kb;
      vs[j * D + jp] = v_a[p];
      vs[j * D + jp + half] = v_b[p];
      if (j == r) {
        qs[jp] = rp.qa;
        qs[jp + half] = rp.qb;
        if (in_cache) {
          const int64_t rr = pos_r * D;
          K[rr + jp] = rp.ka;
          K[rr + jp + half] = rp.kb;
          V[rr + jp] = v_a[p];
          V[rr + jp + half] = v_b[p];
        }
      }
    }
  }
  __syncthreads();  // qs, ks and vs, written above, are read below
  // positions pos0 .. pos0 + r (those >= 0) from LDS: ks row t - pos0
  // (positions at or beyond max_len are not in the cache: none of them is read)
  const int64_t lo = pos0 < 0 ? 0 : pos0;
  const bool sub = lo <= pos_r && lo < max_len;
  const int64_t off = sub ? (lo - pos0) * D : 0;
  att.run(qs, ks + off, vs + off, sub ? static_cast<int>(lo) : INT_MAX, scale, sc, red_m, red_l, part,
          out + static_cast<int64_t>(r) * H + static_cast<int64_t>(h) * D);
}

// Launches of the attention kernels for head_dim = 8 * LPR (LPR = 1, 2, 4, 8, 16 or 32).
template <int LPR>
void launch_attention(const void* q, const void* kc, const void* vc, const int64_t* pos, void* out, int heads,
                      int rows, int max_len, float scale, hipStream_t st) {
  attention_kernel<LPR><<<dim3(heads, rows), kAttnThreads, 0, st>>>(static_cast<const uint16_t*>(q),
                                                        static_cast<const uint16_t*>(kc),
                                                        static_cast<const uint16_t*>(vc), pos,
                                                        static_cast<uint16_t*>(out), max_len, scale);
}

template <int LPR>
void launch_rope_attention(const void* qkv, const void* qw, const void* kw, const float* inv_freq, const int64_t* pos,
                           void* kc, void* vc, void* out, int heads, int rows, int max_len, float eps, float scale,
                           hipStream_t st) {
  if (rows == 1) {
    rope_attention_kernel<LPR><<<heads, kAttnThreads, 0, st>>>(
        static_cast<const uint16_t*>(qkv), static_cast<const uint16_t*>(qw), static_cast<const uint16_t*>(kw),
        inv_freq, pos, static_cast<uint16_t*>(kc), static_cast<uint16_t*>(vc), static_cast<uint16_t*>(out), heads,
        max_len, eps, scale);
  } else {
    rope_attention_rows_kernel<LPR><<<dim3(heads, rows), kAttnThreads, 0, st>>>(
        static_cast<const uint16_t*>(qkv), static_cast<const uint16_t*>(qw), static_cast<const uint16_t*>(kw),
        inv_freq, pos, static_cast<uint16_t*>(kc), static_cast<uint16_t*>(vc), static_cast<uint16_t*>(out), heads,
        max_len, eps, scale);
  }
}

constexpr int kNormMax = 16384;  // elements of one norm row (its bf16 copy in LDS: 32 KiB)

// The row x (bf16 values in LDS) normalised: out = bf16(residual + bf16(w * (x * r))), r = 1 / sqrt(mean(x^2) +
// eps), the mean square in wave_sumsq's order (every wave computes it).
__device__ __forceinline__ void norm_row_out(const uint16_t* xs, const uint16_t* __restrict__ w,
                                             const uint16_t* residual, uint16_t* out, int n, float eps) {
  const float ss = wave_sumsq_lds(xs, n);
  const float r = 1.f / sqrtf(ss / static_cast<float>(n) + eps);
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float y = round_to_bf16(ld_bf16(w, i) * (bf16_bits_to_float(xs[i]) * r));
    out[i] = float_to_bf16_bits(residual != nullptr ? ld_bf16(residual, i) + y : y);
  }
}

// grid = rows, one workgroup per row of x / residual / out [rows, n], n <= kNormMax; out may alias residual.
__global__ __launch_bounds__(kBlock) void norm_residual_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ w,
                                                               const uint16_t* residual, uint16_t* out, int n,
                                                               float eps) {
  extern __shared__ uint16_t norm_xs[];
  const int64_t row = static_cast<int64_t>(blockIdx.x) * n;
  for (int i = threadIdx.x; i < n; i += blockDim.x) norm_xs[i] = x[row + i];
  __syncthreads();
  norm_row_out(norm_xs, w, residual != nullptr ? residual + row : nullptr, out + row, n, eps);
}

// norm_residual_kernel's arithmetic, bit for bit, for rows of n % 8 == 0 elements with 16-byte aligned x, w,
// residual and out: a thread owns pieces of 8 elements (one 16-byte load each of x, w and the residual, every load
// issued before the barrier), so the launch makes one memory round trip before its sum of squares instead of two.
constexpr int kNormVecThreads = 256;
constexpr int kNormVecPer = kNormMax / 8 / kNormVecThreads;  // pieces per thread at the longest row

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

__global__ __launch_bounds__(kNormVecThreads) void norm_residual_vec_kernel(const uint16_t* __restrict__ x,
                                                                            const uint16_t* __restrict__ w,
                                                                            const uint16_t* residual, uint16_t* out,
                                                                            int n, float eps) {
  extern __shared__ uint16_t norm_xs[];
  const int64_t row = static_cast<int64_t>(blockIdx.x) * n;
  const int pieces = n / 8;
  const bool res = residual != nullptr;
  uint4 xv[kNormVecPer], wv[kNormVecPer], rv[kNormVecPer];
#pragma unroll
  for (int j = 0; j < kNormVecPer; ++j) {
    const int p = static_cast<int>(threadIdx.x) + j * kNormVecThreads;
    if (p < pieces) {
      xv[j] = *reinterpret_cast<const uint4*>(x + row + 8 * p);
      wv[j] = *reinterpret_cast<const uint4*>(w + 8 * p);
      rv[j] = res ? *reinterpret_cast<const uint4*>(residual + row + 8 * p) : uint4{0u, 0u, 0u, 0u};
    }
  }
#pragma unroll
  for (int j = 0; j < kNormVecPer; ++j) {
    const int p = static_cast<int>(threadIdx.x) + j * kNormVecThreads;
    if (p < pieces) *reinterpret_cast<uint4*>(norm_xs + 8 * p) = xv[j];
  }
  __syncthreads();
  const float ss = wave_sumsq_lds(norm_xs, n);
  const float r = 1.f / sqrtf(ss / static_cast<float>(n) + eps);
#pragma unroll
  for (int j = 0; j < kNormVecPer; ++j) {
    const int p = static_cast<int>(threadIdx.x) + j * kNormVecThreads;
    if (p < pieces) {
      const uint32_t xa[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
      const uint32_t wa[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
      const uint32_t ra[4] = {rv[j].x, rv[j].y, rv[j].z, rv[j].w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float y0 = round_to_bf16(bf16_lo(wa[e]) * (bf16_lo(xa[e]) * r));
        const float y1 = round_to_bf16(bf16_hi(wa[e]) * (bf16_hi(xa[e]) * r));
        const uint32_t o0 = float_to_bf16_bits(res ? bf16_lo(ra[e]) + y0 : y0);
        const uint32_t o1 = float_to_bf16_bits(res ? bf16_hi(ra[e]) + y1 : y1);
        o[e] = o0 | (o1 << 16);
      }
      *reinterpret_cast<uint4*>(out + row + 8 * p) = uint4{o[0], o[1], o[2], o[3]};
    }
  }
}

// The split-K reduce of a projection's partials (ws [split][rows][n], added in split order, the int8 scale applied
// to the sum, rounded to bf16: splitk_reduce_kernel's arithmetic) feeding norm_residual_kernel's arithmetic in the
// same workgroup (grid = rows, n <= kNormMax): out = bf16(residual + bf16(w * y * rsqrt(mean(y^2) + eps))), equal
// bit for bit to the two launches; out may alias residual.
__global__ __launch_bounds__(kBlock) void splitk_norm_residual_kernel(const float* __restrict__ ws, int split,
                                                                      const void* __restrict__ scale, int scale_dt,
                                                                      const uint16_t* __restrict__ w,
                                                                      const uint16_t* residual, uint16_t* out, int n,
                                                                      float eps) {
  extern __shared__ uint16_t norm_xs[];
  const int64_t total = static_cast<int64_t>(gridDim.x) * n;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * n;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    float t = ws[row + i];
    for (int s = 1; s < split; ++s) t += ws[s * total + row + i];
    if (scale != nullptr) t *= load_scale(scale, i, scale_dt);
    norm_xs[i] = float_to_bf16_bits(t);
  }
  __syncthreads();
  norm_row_out(norm_xs, w, residual != nullptr ? residual + row : nullptr, out + row, n, eps);
}

// out[r, f] = bf16(bf16(silu(g)) * u) for rows r of gu [rows, 2F]: g = gu[r, f], u = gu[r, F + f] (concatenated
// halves) or g = gu[r, 2f], u = gu[r, 2f + 1] (interleaved rows of the weight).
__global__ void silu_mul_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out, int F, int rows,
                                int interleaved) {
  const int64_t total = static_cast<int64_t>(rows) * F;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / F, f = i % F;
    const uint16_t* g2 = gu + r * 2 * F;
    const float g = interleaved ? ld_bf16(g2, 2 * f) : ld_bf16(g2, f);
    const float u = interleaved ? ld_bf16(g2, 2 * f + 1) : ld_bf16(g2, F + f);
    const float a = round_to_bf16(g / (1.f + expf(-g)));
    out[i] = float_to_bf16_bits(a * u);
  }
}

// (value, index) order of torch.argmax: NaN first, then the larger value, then the smaller index.
__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na != nb) return na;
  if (!na && a != b) return a > b;
  return ia < ib;
}

constexpr int kArgmaxBlocks = 64;    // workgroups of argmax_next
constexpr long kArgmaxSpin = 1L << 16;  // re-reads of a stale partial word before the fold gives up on it
constexpr int kArgmaxThreads = 256;  // threads per workgroup

// (best value, index) of this thread folded with (v, i).
__device__ __forceinline__ void take(float& best, int& idx, float v, int i) {
  if (better(v, i, best, idx)) {
    best = v;
    idx = i;
  }
}

// Wave-wide fold of (best, idx): every lane ends with the wave's result.
__device__ __forceinline__ void wave_take(float& best, int& idx) {
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o);
    const int oi = __shfl_xor(idx, o);
    take(best, idx, ov, oi);
  }
}

// scratch words (u32) per row: the partials [kArgmaxBlocks] as 64-bit words, then the launch generation, the
// ticket counter, the error word (set to 1 by a fold that gave up on a stale partial) and one word of padding (the
// next row's partials stay 8-byte aligned)
constexpr int kArgmaxWordGen = 2 * kArgmaxBlocks;
constexpr int kArgmaxWordError = kArgmaxWordGen + 2;
constexpr int kArgmaxRowWords = kArgmaxWordGen + 4;
static_assert(kArgmaxRowWords == BP_ARGMAX_ROW_WORDS && kArgmaxWordError == BP_ARGMAX_ERROR_WORD, "header layout");

// The 16-bit tag of launch generation gen: never 0 (zeroed words are stale), and consecutive generations differ
// even where the 32-bit generation wraps (the period 2^15 divides 2^32).
__device__ __forceinline__ uint32_t argmax_tag(uint32_t gen) { return (gen & 0x7fffu) + 1u; }

// grid = (G, rows), G <= kArgmaxBlocks: for row r of logits [rows, V], G workgroups each take an even share
// (vec: 16-byte aligned rows, 8 logits per load; the V % 8 tail and, when not vec, every element one at a time);
// each stores its (value, index) to the row's scratch as one 64-bit word [tag 16 : bf16 value 16 : index 32] with
// an agent-scope (device-coherent) store, no fence, then takes a ticket; the last workgroup of the row reads the
// words (re-reading any whose tag is not the launch's), folds them and writes tok[r]; with pos (one row only), it
// also advances *pos. The tag is argmax_tag of the row's generation (advanced by that last workgroup, after every
// other workgroup read it). A word still stale after kArgmaxSpin re-reads sets the row's error word (the token is
// then not to be trusted; the host reads the word, nothing clears it). The logits are bf16, so a partial's value
// is exact in 16 bits. better() is a total order, so the result does not depend on the split. Scratch per row:
// the words, the generation, the counter, the error word (all zero before the first launch; the counter is left at
// zero).
__global__ __launch_bounds__(kArgmaxThreads) void argmax_next_kernel(const uint16_t* __restrict__ logits, int V,
                                                                     int vec, int64_t* __restrict__ tok,
                                                                     int64_t* __restrict__ pos,
                                                                     uint32_t* __restrict__ scratch) {
  __shared__ float bv[kArgmaxThreads / kWave];
  __shared__ int bi[kArgmaxThreads / kWave];
  __shared__ uint32_t ticket;
  const int row = blockIdx.y;
  logits += static_cast<int64_t>(row) * V;
  scratch += static_cast<int64_t>(row) * kArgmaxRowWords;
  uint64_t* words = reinterpret_cast<uint64_t*>(scratch);
  uint32_t* gen_p = scratch + kArgmaxWordGen;
  uint32_t* counter = gen_p + 1;
  uint32_t* error = scratch + kArgmaxWordError;
  const int b = blockIdx.x, G = gridDim.x;
  // the launch's generation, read before the ticket (only the last workgroup advances it, after every ticket)
  const uint32_t gen = threadIdx.x == 0 ? __hip_atomic_load(as_global(gen_p), __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT) : 0u;
  float best = -INFINITY;
  int idx = 0x7fffffff;
  const int nvec = vec ? V / 8 : 0;
  const int c_lo = static_cast<int>(static_cast<int64_t>(nvec) * b / G);
  const int c_hi = static_cast<int>(static_cast<int64_t>(nvec) * (b + 1) / G);
  for (int c0 = c_lo + static_cast<int>(threadIdx.x); c0 < c_hi; c0 += 4 * blockDim.x) {
    u32x4 w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = c0 + u * static_cast<int>(blockDim.x);
      w[u] = u32x4{0u, 0u, 0u, 0u};
      if (c < c_hi) w[u] = *reinterpret_cast<const u32x4*>(logits + 8 * static_cast<int64_t>(c));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = c0 + u * static_cast<int>(blockDim.x);
      if (c < c_hi) {
        const uint32_t wd[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          take(best, idx, bf16_bits_to_float(wd[e] & 0xffffu), 8 * c + 2 * e);
          take(best, idx, bf16_bits_to_float(wd[e] >> 16), 8 * c + 2 * e + 1);
        }
      }
    }
  }
  // elements past the vectors: an even share per workgroup
  const int rest = V - 8 * nvec;
  const int e_lo = 8 * nvec + static_cast<int>(static_cast<int64_t>(rest) * b / G);
  const int e_hi = 8 * nvec + static_cast<int>(static_cast<int64_t>(rest) * (b + 1) / G);
  for (int i = e_lo + static_cast<int>(threadIdx.x); i < e_hi; i += blockDim.x) take(best, idx, ld_bf16(logits, i), i);
  wave_take(best, idx);
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) {
    bv[wave] = best;
    bi[wave] = idx;
  }
  __syncthreads();
  __shared__ uint32_t tag_s;
  if (threadIdx.x == 0) {
    for (int w = 0; w < static_cast<int>(blockDim.x / kWave); ++w) take(best, idx, bv[w], bi[w]);
    const uint32_t tag = argmax_tag(gen);
    tag_s = tag;
    // best is -inf (no element) or a bf16 logit: its upper 16 bits hold it exactly
    const uint64_t word = (static_cast<uint64_t>(tag) << 48) | (static_cast<uint64_t>(__float_as_uint(best) >> 16)
                                                                 << 32) | static_cast<uint32_t>(idx);
    __hip_atomic_store(as_global_mut(words + b), word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ticket = __hip_atomic_fetch_add(as_global_mut(counter), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (ticket != static_cast<uint32_t>(G - 1) || threadIdx.x >= kWave) return;
  const uint32_t tag = tag_s;
  best = -INFINITY;
  idx = 0x7fffffff;
  for (int k = threadIdx.x; k < G; k += kWave) {
    uint64_t w = __hip_atomic_load(as_global(words + k), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (long spin = 0; static_cast<uint32_t>(w >> 48) != tag; ++spin) {
      if (spin == kArgmaxSpin) {
        __hip_atomic_store(as_global_mut(error), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      w = __hip_atomic_load(as_global(words + k), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    take(best, idx, __uint_as_float(static_cast<uint32_t>(w >> 16) & 0xffff0000u), static_cast<int>(w));
  }
  wave_take(best, idx);
  if (threadIdx.x == 0) {
    tok[row] = idx == 0x7fffffff ? 0 : idx;
    if (pos != nullptr) *pos += 1;
    __hip_atomic_store(as_global_mut(counter), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(as_global_mut(gen_p), gen + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}

}  // namespace
}  // namespace bp

extern "C" {

int bp_decode_embed_rows(const int64_t* tok, const void* table, void* x, int rows, int hidden, int64_t vocab,
                         void* stream) {
  if (tok == nullptr || table == nullptr || x == nullptr || rows <= 0 || hidden <= 0 || vocab <= 0)
    return BP_E_INVALID_ARG;
  bp::embed_kernel<<<rows, bp::kBlock, 0, static_cast<hipStream_t>(stream)>>>(
      tok, static_cast<const uint16_t*>(table), static_cast<uint16_t*>(x), hidden, vocab);
  return bp::status();
}

int bp_decode_embed(const int64_t* tok, const void* table, void* x, int hidden, int64_t vocab, void* stream) {
  if (tok == nullptr || table == nullptr || x == nullptr || hidden <= 0 || vocab <= 0) return BP_E_INVALID_ARG;
  bp::embed_kernel<<<1, bp::kBlock, 0, static_cast<hipStream_t>(stream)>>>(
      tok, static_cast<const uint16_t*>(table), static_cast<uint16_t*>(x), hidden, vocab);
  return bp::status();
}

int bp_decode_qk_rope_cache_rows(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                                 const int64_t* pos, void* q_out, void* k_cache, void* v_cache, int heads,
                                 int head_dim, int max_len, float eps, int rows, void* stream) {
  if (qkv == nullptr || q_norm_w == nullptr || k_norm_w == nullptr || inv_freq == nullptr || pos == nullptr ||
      q_out == nullptr || k_cache == nullptr || v_cache == nullptr || heads <= 0 || max_len <= 0 || rows <= 0)
    return BP_E_INVALID_ARG;
  if (head_dim <= 0 || head_dim % 8 != 0) return BP_E_UNSUPPORTED;
  if (!bp::aligned16(qkv)) return BP_E_INVALID_ARG;
  bp::qk_rope_cache_kernel<<<rows, bp::kAttnThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(qkv), static_cast<const uint16_t*>(q_norm_w),
      static_cast<const uint16_t*>(k_norm_w), inv_freq, pos, static_cast<uint16_t*>(q_out),
      static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), heads, head_dim, max_len, eps);
  return bp::status();
}

int bp_decode_qk_rope_cache(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                            const int64_t* pos, void* q_out, void* k_cache, void* v_cache, int heads, int head_dim,
                            int max_len, float eps, void* stream) {
  return bp_decode_qk_rope_cache_rows(qkv, q_norm_w, k_norm_w, inv_freq, pos, q_out, k_cache, v_cache, heads,
                                      head_dim, max_len, eps, 1, stream);
}

int bp_decode_attention(const void* q, const void* k_cache, const void* v_cache, const int64_t* pos, void* out,
                        int heads, int head_dim, int max_len, float scale, void* stream) {
  return bp_decode_attention_rows(q, k_cache, v_cache, pos, out, heads, head_dim, max_len, scale, 1, stream);
}

int bp_decode_attention_rows(const void* q, const void* k_cache, const void* v_cache, const int64_t* pos, void* out,
                             int heads, int head_dim, int max_len, float scale, int rows, void* stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr || pos == nullptr || out == nullptr || heads <= 0 ||
      max_len <= 0 || rows <= 0)
    return BP_E_INVALID_ARG;
  if (head_dim <= 0 || head_dim % 8 != 0 || head_dim > 256 || bp::kAttnThreads % head_dim != 0 ||
      max_len > bp::kAttnMaxLen)
    return BP_E_UNSUPPORTED;
  if (!bp::aligned16(k_cache) || !bp::aligned16(v_cache)) return BP_E_INVALID_ARG;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (head_dim / 8) {
    case 1: bp::launch_attention<1>(q, k_cache, v_cache, pos, out, heads, rows, max_len, scale, st); break;
    case 2: bp::launch_attention<2>(q, k_cache, v_cache, pos, out, heads, rows, max_len, scale, st); break;
    case 4: bp::launch_attention<4>(q, k_cache, v_cache, pos, out, heads, rows, max_len, scale, st); break;
    case 8: bp::launch_attention<8>(q, k_cache, v_cache, pos, out, heads, rows, max_len, scale, st); break;
    case 16: bp::launch_attention<16>(q, k_cache, v_cache, pos, out, heads, rows, max_len, scale, st); break;
    case 32: bp::launch_attention<32>(q, k_cache, v_cache, pos, out, heads, rows, max_len, scale, st); break;
    default: return BP_E_UNSUPPORTED;
  }
  return bp::status();
}

int bp_decode_rope_attention(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                             const int64_t* pos, void* k_cache, void* v_cache, void* out, int heads, int head_dim,
                             int max_len, float eps, float scale, void* stream) {
  return bp_decode_rope_attention_rows(qkv, q_norm_w, k_norm_w, inv_freq, pos, k_cache, v_cache, out, heads, head_dim,
                                       1, max_len, eps, scale, stream);
}

int bp_decode_rope_attention_rows(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                                  const int64_t* pos, void* k_cache, void* v_cache, void* out, int heads, int head_dim,
                                  int rows, int max_len, float eps, float scale, void* stream) {
  if (qkv == nullptr || q_norm_w == nullptr || k_norm_w == nullptr || inv_freq == nullptr || pos == nullptr ||
      k_cache == nullptr || v_cache == nullptr || out == nullptr || heads <= 0 || max_len <= 0 || rows <= 0)
    return BP_E_INVALID_ARG;
  if (rows > bp::kRowsMax) return BP_E_UNSUPPORTED;
  if (head_dim <= 0 || head_dim % 8 != 0 || head_dim > 256 || bp::kAttnThreads % head_dim != 0 ||
      max_len > bp::kAttnMaxLen)
    return BP_E_UNSUPPORTED;
  if (!bp::aligned16(qkv) || !bp::aligned16(k_cache) || !bp::aligned16(v_cache)) return BP_E_INVALID_ARG;
  // the verify launch reads its rows of q|k|v through one buffer resource (under 2^31 bytes)
  if (static_cast<int64_t>(rows) * 3 * heads * head_dim * 2 >= (int64_t{1} << 31)) return BP_E_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
#define BP_ROPE_ATT(L)                                                                                           \
  bp::launch_rope_attention<L>(qkv, q_norm_w, k_norm_w, inv_freq, pos, k_cache, v_cache, out, heads, rows, max_len, \
                               eps, scale, st)
  switch (head_dim / 8) {
    case 1: BP_ROPE_ATT(1); break;
    case 2: BP_ROPE_ATT(2); break;
    case 4: BP_ROPE_ATT(4); break;
    case 8: BP_ROPE_ATT(8); break;
    case 16: BP_ROPE_ATT(16); break;
    case 32: BP_ROPE_ATT(32); break;
    default: return BP_E_UNSUPPORTED;
  }
#undef BP_ROPE_ATT
  return bp::status();
}

int bp_decode_norm_residual_rows(const void* x, const void* weight, const void* residual, void* out, int n,
                                 float eps, int rows, void* stream) {
  if (x == nullptr || weight == nullptr || out == nullptr || n <= 0 || rows <= 0) return BP_E_INVALID_ARG;
  if (n > bp::kNormMax) return BP_E_UNSUPPORTED;
  using bp::aligned16;
  if (n % 8 == 0 && aligned16(x) && aligned16(weight) && aligned16(out) &&
      (residual == nullptr || aligned16(residual)))
    bp::norm_residual_vec_kernel<<<rows, bp::kNormVecThreads, static_cast<size_t>(n) * 2,
                                   static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(weight),
        static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out), n, eps);
  else
    bp::norm_residual_kernel<<<rows, bp::kBlock, static_cast<size_t>(n) * 2, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(weight),
        static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out), n, eps);
  return bp::status();
}

int bp_decode_splitk_norm_residual_rows(const float* workspace, int split, const void* scale, int scale_dtype,
                                        const void* weight, const void* residual, void* out, int n, float eps,
                                        int rows, void* stream) {
  if (workspace == nullptr || weight == nullptr || out == nullptr || n <= 0 || rows <= 0 || split < 1)
    return BP_E_INVALID_ARG;
  if (scale != nullptr && (scale_dtype < BP_DT_BF16 || scale_dtype > BP_DT_F32)) return BP_E_INVALID_ARG;
  if (n > bp::kNormMax) return BP_E_UNSUPPORTED;
  bp::splitk_norm_residual_kernel<<<rows, bp::kBlock, static_cast<size_t>(n) * 2,
                                    static_cast<hipStream_t>(stream)>>>(
      workspace, split, scale, scale_dtype, static_cast<const uint16_t*>(weight),
      static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out), n, eps);
  return bp::status();
}

int bp_decode_norm_residual(const void* x, const void* weight, const void* residual, void* out, int n, float eps,
                            void* stream) {
  return bp_decode_norm_residual_rows(x, weight, residual, out, n, eps, 1, stream);
}

int bp_decode_silu_mul_rows(const void* gate_up, void* out, int ffn, int rows, int interleaved, void* stream) {
  if (gate_up == nullptr || out == nullptr || ffn <= 0 || rows <= 0) return BP_E_INVALID_ARG;
  const int64_t total = static_cast<int64_t>(ffn) * rows;
  const int blocks = static_cast<int>((total + 255) / 256 < 1024 ? (total + 255) / 256 : 1024);
  bp::silu_mul_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), ffn, rows, interleaved ? 1 : 0);
  return bp::status();
}

int bp_decode_silu_mul(const void* gate_up, void* out, int ffn, void* stream) {
  return bp_decode_silu_mul_rows(gate_up, out, ffn, 1, 0, stream);
}

size_t bp_decode_argmax_scratch_bytes(void) { return bp::kArgmaxRowWords * sizeof(uint32_t); }

size_t bp_decode_argmax_rows_scratch_bytes(int rows) {
  return rows <= 0 ? 0 : static_cast<size_t>(rows) * bp::kArgmaxRowWords * sizeof(uint32_t);
}

int bp_decode_argmax_next(const void* logits, int vocab, int64_t* tok, int64_t* pos, void* scratch, void* stream) {
  if (logits == nullptr || tok == nullptr || pos == nullptr || scratch == nullptr || vocab <= 0 ||
      reinterpret_cast<uintptr_t>(scratch) % 8 != 0)
    return BP_E_INVALID_ARG;
  bp::argmax_next_kernel<<<dim3(bp::kArgmaxBlocks, 1), bp::kArgmaxThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(logits), vocab, bp::aligned16(logits) ? 1 : 0, tok, pos,
      static_cast<uint32_t*>(scratch));
  return bp::status();
}

int bp_decode_argmax_rows(const void* logits, int vocab, int rows, int64_t* tok, void* scratch, void* stream) {
  if (logits == nullptr || tok == nullptr || scratch == nullptr || vocab <= 0 || rows <= 0 ||
      reinterpret_cast<uintptr_t>(scratch) % 8 != 0)
    return BP_E_INVALID_ARG;
  const int vec = bp::aligned16(logits) && (rows == 1 || vocab % 8 == 0) ? 1 : 0;
  // about kArgmaxBlocks workgroups in all: the last one of a row reads every partial (the result does not depend
  // on the split: the fold is exact)
  const int per_row = bp::kArgmaxBlocks / rows > 4 ? bp::kArgmaxBlocks / rows : 4;
  bp::argmax_next_kernel<<<dim3(per_row, rows), bp::kArgmaxThreads, 0,
                           static_cast<hipStream_t>(stream)>>>(static_cast<const uint16_t*>(logits), vocab, vec, tok,
                                                               nullptr, static_cast<uint32_t*>(scratch));
  return bp::status();
}

}  // extern "C"
