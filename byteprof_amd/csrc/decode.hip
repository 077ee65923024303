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
//   norm_residual   out <- bf16(residual + bf16(w * x * rsqrt(mean(x^2) + eps))) (no residual: the plain norm)
//   silu_mul        out <- bf16(bf16(silu(g)) * u), g and u the two halves of the fused gate|up projection
//   argmax_next     tok <- first index of the largest logit (NaN counts as largest); pos <- pos + 1
//
// The roundings are those of transformers' Olmo2ForCausalLM run in bf16 with the eager attention, the model whose
// forward the reference's decode loop replays (byteprof/optim/olmo.py:122-219: make_generate_graph captures the
// forward, the argmax and the next-step input updates in one graph).

#include "byteprof_amd.h"
#include "common.h"

namespace bp {
namespace {

constexpr int kBlock = 1024;       // threads of the one-workgroup kernels
constexpr int kAttnThreads = 256;  // threads per head in the attention
constexpr int kAttnMaxLen = 4096;  // positions a cache may hold (scores in LDS)

// Sum of v over the workgroup (blockDim.x a multiple of 64, at most kBlock); every thread gets the total.
__device__ float block_sum(float v, float* red) {
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, waves = blockDim.x / kWave;
  __syncthreads();  // red may still be read by a previous call
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < waves; ++i) t += red[i];
  return t;
}

__device__ float block_max(float v, float* red) {
  for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, waves = blockDim.x / kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
  for (int i = 1; i < waves; ++i) t = fmaxf(t, red[i]);
  return t;
}

__device__ __forceinline__ float ld_bf16(const uint16_t* p, int64_t i) { return bf16_bits_to_float(p[i]); }

__global__ __launch_bounds__(kBlock) void embed_kernel(const int64_t* __restrict__ tok,
                                                       const uint16_t* __restrict__ table,
                                                       uint16_t* __restrict__ x, int H, int64_t V) {
  int64_t t = *tok;
  t = t < 0 ? 0 : (t >= V ? V - 1 : t);  // ids are validated on the host; the clamp keeps the read in bounds
  for (int i = threadIdx.x; i < H; i += blockDim.x) x[i] = table[t * H + i];
}

// One workgroup; thread t owns the RoPE pairs (h, j), (h, j + D/2) of q and of k for pair index i = t, t + block..
__global__ __launch_bounds__(kBlock) void qk_rope_cache_kernel(const uint16_t* __restrict__ qkv,
                                                               const uint16_t* __restrict__ qw,
                                                               const uint16_t* __restrict__ kw,
                                                               const float* __restrict__ inv_freq,
                                                               const int64_t* __restrict__ pos_p,
                                                               uint16_t* __restrict__ q_out,
                                                               uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                               int heads, int D, int max_len, float eps) {
  __shared__ float red[kBlock / kWave];
  const int H = heads * D, half = D / 2;
  const int64_t pos = *pos_p;
  const bool in_cache = pos >= 0 && pos < max_len;
  const uint16_t* q = qkv;
  const uint16_t* k = qkv + H;
  const uint16_t* v = qkv + 2 * H;
  float sq = 0.f, sk = 0.f;
  for (int i = threadIdx.x; i < H / 2; i += blockDim.x) {
    const int h = i / half, j = i % half;
    const float qa = ld_bf16(q, h * D + j), qb = ld_bf16(q, h * D + j + half);
    const float ka = ld_bf16(k, h * D + j), kb = ld_bf16(k, h * D + j + half);
    sq += qa * qa + qb * qb;
    sk += ka * ka + kb * kb;
  }
  const float rq = 1.f / sqrtf(block_sum(sq, red) / static_cast<float>(H) + eps);
  const float rk = 1.f / sqrtf(block_sum(sk, red) / static_cast<float>(H) + eps);
  for (int i = threadIdx.x; i < H / 2; i += blockDim.x) {
    const int h = i / half, j = i % half;
    const int a = h * D + j, b = a + half;
    const float f = inv_freq[j] * static_cast<float>(pos);
    const float c = cosf(f), s = sinf(f);
    const float qa = round_to_bf16(ld_bf16(qw, a) * (ld_bf16(q, a) * rq));
    const float qb = round_to_bf16(ld_bf16(qw, b) * (ld_bf16(q, b) * rq));
    const float ka = round_to_bf16(ld_bf16(kw, a) * (ld_bf16(k, a) * rk));
    const float kb = round_to_bf16(ld_bf16(kw, b) * (ld_bf16(k, b) * rk));
    q_out[a] = float_to_bf16_bits(qa * c + (-qb) * s);
    q_out[b] = float_to_bf16_bits(qb * c + qa * s);
    if (in_cache) {
      const int64_t row = (static_cast<int64_t>(h) * max_len + pos) * D;
      kc[row + j] = float_to_bf16_bits(ka * c + (-kb) * s);
      kc[row + j + half] = float_to_bf16_bits(kb * c + ka * s);
      vc[row + j] = v[a];
      vc[row + j + half] = v[b];
    }
  }
}

// grid = heads; positions 0 .. pos of the head's cache rows [max_len, D].
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(const uint16_t* __restrict__ q,
                                                                 const uint16_t* __restrict__ kc,
                                                                 const uint16_t* __restrict__ vc,
                                                                 const int64_t* __restrict__ pos_p,
                                                                 uint16_t* __restrict__ out, int D, int max_len,
                                                                 float scale) {
  __shared__ float sc[kAttnMaxLen];
  __shared__ float qs[512];
  __shared__ float red[kAttnThreads / kWave];
  __shared__ float part[kAttnThreads];
  const int h = blockIdx.x;
  int64_t pos = *pos_p;
  pos = pos < 0 ? 0 : (pos >= max_len ? max_len - 1 : pos);
  const int T = static_cast<int>(pos) + 1;
  for (int d = threadIdx.x; d < D; d += blockDim.x) qs[d] = ld_bf16(q, static_cast<int64_t>(h) * D + d);
  __syncthreads();
  const uint16_t* K = kc + static_cast<int64_t>(h) * max_len * D;
  const uint16_t* V = vc + static_cast<int64_t>(h) * max_len * D;
  float m = -INFINITY;
  for (int t = threadIdx.x; t < T; t += blockDim.x) {
    const uint16_t* kr = K + static_cast<int64_t>(t) * D;
    float dot = 0.f;
    for (int d = 0; d < D; d += 8) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(kr + d);
      const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dot += bf16_bits_to_float(wd[e] & 0xffffu) * qs[d + 2 * e];
        dot += bf16_bits_to_float(wd[e] >> 16) * qs[d + 2 * e + 1];
      }
    }
    const float s = round_to_bf16(round_to_bf16(dot) * scale);
    sc[t] = s;
    m = fmaxf(m, s);
  }
  m = block_max(m, red);
  float l = 0.f;
  for (int t = threadIdx.x; t < T; t += blockDim.x) {
    const float e = expf(sc[t] - m);
    sc[t] = e;
    l += e;
  }
  l = block_sum(l, red);  // its barriers also order the sc writes before the reads below
  const float inv = 1.f / l;
  // thread (d, r): dimension d, positions t = r, r + R, ... (R = blockDim.x / D rows of threads)
  const int R = blockDim.x / D;
  const int d = threadIdx.x % D, r = threadIdx.x / D;
  float acc = 0.f;
  if (r < R) {
    for (int t = r; t < T; t += R) acc += round_to_bf16(sc[t] * inv) * ld_bf16(V, static_cast<int64_t>(t) * D + d);
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x < D) {
    float t = 0.f;
    for (int i = 0; i < R; ++i) t += part[i * D + threadIdx.x];
    out[static_cast<int64_t>(h) * D + threadIdx.x] = float_to_bf16_bits(t);
  }
}

// qk_rope_cache and attention in one launch: every workgroup h computes the q / k norms over the whole projections
// (the same sums in every workgroup; their summation order differs from qk_rope_cache_kernel's, so a value may land
// one bf16 step apart), rotates its own head, writes its k and v at pos, and attends over positions 0 .. pos.
__global__ __launch_bounds__(kAttnThreads) void rope_attention_kernel(const uint16_t* __restrict__ qkv,
                                                                      const uint16_t* __restrict__ qw,
                                                                      const uint16_t* __restrict__ kw,
                                                                      const float* __restrict__ inv_freq,
                                                                      const int64_t* __restrict__ pos_p,
                                                                      uint16_t* __restrict__ kc,
                                                                      uint16_t* __restrict__ vc,
                                                                      uint16_t* __restrict__ out, int heads, int D,
                                                                      int max_len, float eps, float scale) {
  __shared__ float sc[kAttnMaxLen];
  __shared__ float qs[512];
  __shared__ float red[kAttnThreads / kWave];
  __shared__ float part[kAttnThreads];
  const int h = blockIdx.x;
  const int H = heads * D, half = D / 2;
  const int64_t pos_in = *pos_p;
  const bool in_cache = pos_in >= 0 && pos_in < max_len;
  const uint16_t* q = qkv;
  const uint16_t* k = qkv + H;
  const uint16_t* v = qkv + 2 * H;
  float sq = 0.f, sk = 0.f;
  for (int i = threadIdx.x; i < H; i += blockDim.x) {
    const float a = ld_bf16(q, i), b = ld_bf16(k, i);
    sq += a * a;
    sk += b * b;
  }
  const float rq = 1.f / sqrtf(block_sum(sq, red) / static_cast<float>(H) + eps);
  const float rk = 1.f / sqrtf(block_sum(sk, red) / static_cast<float>(H) + eps);
  uint16_t* K = kc + static_cast<int64_t>(h) * max_len * D;
  uint16_t* V = vc + static_cast<int64_t>(h) * max_len * D;
  for (int j = threadIdx.x; j < half; j += blockDim.x) {
    const int a = h * D + j, b = a + half;
    const float f = inv_freq[j] * static_cast<float>(pos_in);
    const float c = cosf(f), s = sinf(f);
    const float qa = round_to_bf16(ld_bf16(qw, a) * (ld_bf16(q, a) * rq));
    const float qb = round_to_bf16(ld_bf16(qw, b) * (ld_bf16(q, b) * rq));
    const float ka = round_to_bf16(ld_bf16(kw, a) * (ld_bf16(k, a) * rk));
    const float kb = round_to_bf16(ld_bf16(kw, b) * (ld_bf16(k, b) * rk));
    qs[j] = round_to_bf16(qa * c + (-qb) * s);
    qs[j + half] = round_to_bf16(qb * c + qa * s);
    if (in_cache) {
      const int64_t row = pos_in * D;
      K[row + j] = float_to_bf16_bits(ka * c + (-kb) * s);
      K[row + j + half] = float_to_bf16_bits(kb * c + ka * s);
      V[row + j] = v[a];
      V[row + j + half] = v[b];
    }
  }
  __syncthreads();  // qs and this position's cache row, written above, are read below
  const int64_t pos = pos_in < 0 ? 0 : (pos_in >= max_len ? max_len - 1 : pos_in);
  const int T = static_cast<int>(pos) + 1;
  float m = -INFINITY;
  for (int t = threadIdx.x; t < T; t += blockDim.x) {
    const uint16_t* kr = K + static_cast<int64_t>(t) * D;
    float dot = 0.f;
    for (int d = 0; d < D; d += 8) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(kr + d);
      const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dot += bf16_bits_to_float(wd[e] & 0xffffu) * qs[d + 2 * e];
        dot += bf16_bits_to_float(wd[e] >> 16) * qs[d + 2 * e + 1];
      }
    }
    const float s = round_to_bf16(round_to_bf16(dot) * scale);
    sc[t] = s;
    m = fmaxf(m, s);
  }
  m = block_max(m, red);
  float l = 0.f;
  for (int t = threadIdx.x; t < T; t += blockDim.x) {
    const float e = expf(sc[t] - m);
    sc[t] = e;
    l += e;
  }
  l = block_sum(l, red);
  const float inv = 1.f / l;
  const int R = blockDim.x / D;
  const int d = threadIdx.x % D, r = threadIdx.x / D;
  float acc = 0.f;
  for (int t = r; t < T; t += R) acc += round_to_bf16(sc[t] * inv) * ld_bf16(V, static_cast<int64_t>(t) * D + d);
  part[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x < D) {
    float t = 0.f;
    for (int i = 0; i < R; ++i) t += part[i * D + threadIdx.x];
    out[static_cast<int64_t>(h) * D + threadIdx.x] = float_to_bf16_bits(t);
  }
}

__global__ __launch_bounds__(kBlock) void norm_residual_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ w,
                                                               const uint16_t* residual, uint16_t* out, int n,
                                                               float eps) {
  __shared__ float red[kBlock / kWave];
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = ld_bf16(x, i);
    ss += v * v;
  }
  const float r = 1.f / sqrtf(block_sum(ss, red) / static_cast<float>(n) + eps);
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float y = round_to_bf16(ld_bf16(w, i) * (ld_bf16(x, i) * r));
    out[i] = float_to_bf16_bits(residual != nullptr ? ld_bf16(residual, i) + y : y);
  }
}

__global__ void silu_mul_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out, int F) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < F; i += gridDim.x * blockDim.x) {
    const float g = ld_bf16(gu, i);
    const float a = round_to_bf16(g / (1.f + expf(-g)));
    out[i] = float_to_bf16_bits(a * ld_bf16(gu, F + i));
  }
}

// (value, index) order of torch.argmax: NaN first, then the larger value, then the smaller index.
__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na != nb) return na;
  if (!na && a != b) return a > b;
  return ia < ib;
}

__global__ __launch_bounds__(kBlock) void argmax_next_kernel(const uint16_t* __restrict__ logits, int V,
                                                             int64_t* __restrict__ tok, int64_t* __restrict__ pos) {
  __shared__ float bv[kBlock];
  __shared__ int bi[kBlock];
  float best = -INFINITY;
  int idx = 0x7fffffff;
  for (int i = threadIdx.x; i < V; i += blockDim.x) {
    const float v = ld_bf16(logits, i);
    if (better(v, i, best, idx)) {
      best = v;
      idx = i;
    }
  }
  bv[threadIdx.x] = best;
  bi[threadIdx.x] = idx;
  __syncthreads();
  for (int o = blockDim.x / 2; o > 0; o >>= 1) {
    if (threadIdx.x < o && better(bv[threadIdx.x + o], bi[threadIdx.x + o], bv[threadIdx.x], bi[threadIdx.x])) {
      bv[threadIdx.x] = bv[threadIdx.x + o];
      bi[threadIdx.x] = bi[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    *tok = bi[0] == 0x7fffffff ? 0 : bi[0];
    *pos += 1;
  }
}

int status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}

}  // namespace
}  // namespace bp

extern "C" {

int bp_decode_embed(const int64_t* tok, const void* table, void* x, int hidden, int64_t vocab, void* stream) {
  if (tok == nullptr || table == nullptr || x == nullptr || hidden <= 0 || vocab <= 0) return BP_E_INVALID_ARG;
  bp::embed_kernel<<<1, bp::kBlock, 0, static_cast<hipStream_t>(stream)>>>(
      tok, static_cast<const uint16_t*>(table), static_cast<uint16_t*>(x), hidden, vocab);
  return bp::status();
}

int bp_decode_qk_rope_cache(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                            const int64_t* pos, void* q_out, void* k_cache, void* v_cache, int heads, int head_dim,
                            int max_len, float eps, void* stream) {
  if (qkv == nullptr || q_norm_w == nullptr || k_norm_w == nullptr || inv_freq == nullptr || pos == nullptr ||
      q_out == nullptr || k_cache == nullptr || v_cache == nullptr || heads <= 0 || max_len <= 0)
    return BP_E_INVALID_ARG;
  if (head_dim <= 0 || head_dim % 2 != 0) return BP_E_UNSUPPORTED;
  bp::qk_rope_cache_kernel<<<1, bp::kBlock, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(qkv), static_cast<const uint16_t*>(q_norm_w),
      static_cast<const uint16_t*>(k_norm_w), inv_freq, pos, static_cast<uint16_t*>(q_out),
      static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), heads, head_dim, max_len, eps);
  return bp::status();
}

int bp_decode_attention(const void* q, const void* k_cache, const void* v_cache, const int64_t* pos, void* out,
                        int heads, int head_dim, int max_len, float scale, void* stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr || pos == nullptr || out == nullptr || heads <= 0 ||
      max_len <= 0)
    return BP_E_INVALID_ARG;
  if (head_dim <= 0 || head_dim % 8 != 0 || head_dim > 256 || bp::kAttnThreads % head_dim != 0 ||
      max_len > bp::kAttnMaxLen)
    return BP_E_UNSUPPORTED;
  bp::attention_kernel<<<heads, bp::kAttnThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k_cache), static_cast<const uint16_t*>(v_cache),
      pos, static_cast<uint16_t*>(out), head_dim, max_len, scale);
  return bp::status();
}

int bp_decode_rope_attention(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                             const int64_t* pos, void* k_cache, void* v_cache, void* out, int heads, int head_dim,
                             int max_len, float eps, float scale, void* stream) {
  if (qkv == nullptr || q_norm_w == nullptr || k_norm_w == nullptr || inv_freq == nullptr || pos == nullptr ||
      k_cache == nullptr || v_cache == nullptr || out == nullptr || heads <= 0 || max_len <= 0)
    return BP_E_INVALID_ARG;
  if (head_dim <= 0 || head_dim % 8 != 0 || head_dim > 256 || bp::kAttnThreads % head_dim != 0 ||
      max_len > bp::kAttnMaxLen)
    return BP_E_UNSUPPORTED;
  bp::rope_attention_kernel<<<heads, bp::kAttnThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(qkv), static_cast<const uint16_t*>(q_norm_w),
      static_cast<const uint16_t*>(k_norm_w), inv_freq, pos, static_cast<uint16_t*>(k_cache),
      static_cast<uint16_t*>(v_cache), static_cast<uint16_t*>(out), heads, head_dim, max_len, eps, scale);
  return bp::status();
}

int bp_decode_norm_residual(const void* x, const void* weight, const void* residual, void* out, int n, float eps,
                            void* stream) {
  if (x == nullptr || weight == nullptr || out == nullptr || n <= 0) return BP_E_INVALID_ARG;
  bp::norm_residual_kernel<<<1, bp::kBlock, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(weight),
      static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(out), n, eps);
  return bp::status();
}

int bp_decode_silu_mul(const void* gate_up, void* out, int ffn, void* stream) {
  if (gate_up == nullptr || out == nullptr || ffn <= 0) return BP_E_INVALID_ARG;
  const int blocks = (ffn + 255) / 256 < 1024 ? (ffn + 255) / 256 : 1024;
  bp::silu_mul_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), ffn);
  return bp::status();
}

int bp_decode_argmax_next(const void* logits, int vocab, int64_t* tok, int64_t* pos, void* stream) {
  if (logits == nullptr || tok == nullptr || pos == nullptr || vocab <= 0) return BP_E_INVALID_ARG;
  bp::argmax_next_kernel<<<1, bp::kBlock, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(logits), vocab, tok, pos);
  return bp::status();
}

}  // extern "C"
