// C ABI of the library's common entry points (version, status strings, split-K workspace size, the split-K
// reduction) and of the int4 group-128 skinny launch (kernels in skinny_int4.hip). The bf16 / int8 skinny launch
// is skinny_mf.hip.
//
// Reference semantics: byteprof/optim/skinny.py:84-90 (_split_reduce).

#include "byteprof_amd.h"
#include "common.h"
#include "skinny_mf_kernel.h"  // MfPro

namespace bp {

// int4 group-128 kernels (skinny_int4.hip).
using Int4Fn = void (*)(const uint16_t*, const uint8_t*, const void*, int, const uint16_t*, uint16_t*, float*, int,
                        int64_t, int64_t, int);
Int4Fn int4_pick(int mt, int tile_rows, int waves);
using Int4MfFn = void (*)(const uint16_t*, const uint8_t*, const void*, int, const uint16_t*, uint16_t*, float*, int,
                          int64_t, int64_t, int, MfPro);
Int4MfFn int4_mf_pick(int tile_rows, int waves, int scale_dt, int epi, bool pro);

namespace {

__global__ void splitk_reduce_kernel(const float* __restrict__ ws, uint16_t* __restrict__ y,
                                     const void* __restrict__ scale, int scale_dt, int64_t M, int64_t N,
                                     int split) {
  const int64_t total = M * N;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    float t = ws[idx];
    for (int s = 1; s < split; ++s) t += ws[s * total + idx];
    if (scale != nullptr) t *= load_scale(scale, idx % N, scale_dt);
    y[idx] = float_to_bf16_bits(t);
  }
}

// Zero fill with a kernel rather than hipMemsetAsync, so that it is safe inside captured HIP graphs.
__global__ void fill_zero_bf16_kernel(uint16_t* __restrict__ y, int64_t count) {
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < count;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x)
    y[idx] = 0;
}

int row_bucket(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}

int grid_for(int64_t count) {
  const int64_t b = (count + 255) / 256;
  return static_cast<int>(b < 2048 ? (b < 1 ? 1 : b) : 2048);
}

// the prologue's LDS: the rows, gamma, the residual rows and gamma2, (2 M + 2) K bf16 within 64 KiB (K <= 8192 at
// one row, 2048 at up to 7); the per-row sums of squares hold up to 8 rows
constexpr int64_t kInt4ProLdsBytes = 64 * 1024;
constexpr int64_t kInt4ProMaxRows = 8;

// epi 0: y [M, N] (split > 1: partials then the reduce); 1: the gate|up SiLU product y [M, N / 2] of interleaved
// rows (split 1, the matrix-core kernel only). prologue (kind != 0): a transform of the activation rows first
// (split 1, the matrix-core kernel, bf16 scales, M <= 8 and (2 M + 2) K x 2 bytes <= 64 KiB), as bp_skinny_mf_pro's.
int skinny_int4_launch(const void* x, const void* packed, const void* scale, int scale_dt, const void* zero, void* y,
                       int64_t M, int64_t N, int64_t K, int tile_rows, int waves, int split, void* ws,
                       size_t ws_bytes, void* stream, int epi = 0, const BpPrologue* prologue = nullptr) {
  if (M < 0 || N < 0 || K < 0 || M > 16 || K % 128 != 0) return BP_E_INVALID_ARG;
  if (epi != 0 && (split != 1 || N % 2 != 0)) return BP_E_UNSUPPORTED;
  MfPro pro{0, 0.f, nullptr, nullptr, nullptr, 0, nullptr, nullptr};
  if (prologue != nullptr && prologue->kind != 0) {
    if (prologue->kind != BP_PRO_UNIT_RMS && prologue->kind != BP_PRO_NORM) return BP_E_INVALID_ARG;
    if (prologue->kind == BP_PRO_NORM && prologue->gamma == nullptr) return BP_E_INVALID_ARG;
    if (reinterpret_cast<uintptr_t>(prologue->gamma) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(prologue->residual) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(prologue->xout) % 16 != 0 || reinterpret_cast<uintptr_t>(prologue->gamma2) % 16 != 0)
      return BP_E_INVALID_ARG;
    if (prologue->gamma2 != nullptr && prologue->kind != BP_PRO_NORM) return BP_E_INVALID_ARG;
    // workgroup (0, 0) writes xout while the others still read x and the residual row
    const int64_t rows_bytes = 2 * M * K;
    if (ranges_overlap(prologue->xout, rows_bytes, x, rows_bytes) ||
        (prologue->kind == BP_PRO_NORM && ranges_overlap(prologue->xout, rows_bytes, prologue->residual, rows_bytes)))
      return BP_E_INVALID_ARG;
    if (M > kInt4ProMaxRows || split != 1 || (2 * M + 2) * K * 2 > kInt4ProLdsBytes) return BP_E_UNSUPPORTED;
    pro = MfPro{prologue->kind, prologue->eps, static_cast<const uint16_t*>(prologue->gamma),
                static_cast<const uint16_t*>(prologue->residual), static_cast<uint16_t*>(prologue->xout), 1,
                static_cast<const uint16_t*>(prologue->gamma2), nullptr};
  }
  if (M == 0 || N == 0) return BP_OK;
  if (x == nullptr || packed == nullptr || y == nullptr || scale == nullptr || zero == nullptr)
    return BP_E_INVALID_ARG;
  if (scale_dt < BP_DT_BF16 || scale_dt > BP_DT_F32) return BP_E_INVALID_ARG;
  if (split < 1 || split > 1024) return BP_E_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (K == 0) {
    if (pro.kind != 0) return BP_E_UNSUPPORTED;
    // silu(0) * 0 = 0: zeros either way
    const int64_t count = epi != 0 ? M * (N / 2) : M * N;
    fill_zero_bf16_kernel<<<grid_for(count), 256, 0, st>>>(static_cast<uint16_t*>(y), count);
    return launch_status();
  }
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(packed) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(zero) % 2 != 0)
    return BP_E_UNSUPPORTED;
  // the matrix-core kernel where a lane's four rows can read their scale and zero as one vector each, and the
  // activations of up to 16 rows fit one buffer resource (K < 2^24); the choice does not depend on M
  const int64_t sc_align = scale_dt == BP_DT_F32 ? 16 : 8;
  const bool mf = N % 4 == 0 && reinterpret_cast<uintptr_t>(zero) % 8 == 0 &&
                  reinterpret_cast<uintptr_t>(scale) % sc_align == 0 && K < (int64_t{1} << 24);
  if ((epi != 0 || pro.kind != 0) && !mf) return BP_E_UNSUPPORTED;
  Int4MfFn mf_fn = mf ? int4_mf_pick(tile_rows, waves, scale_dt, epi, pro.kind != 0) : nullptr;
  Int4Fn fn = mf ? nullptr : int4_pick(row_bucket(M), tile_rows, waves);
  if (mf_fn == nullptr && fn == nullptr) return BP_E_UNSUPPORTED;
  const int64_t groups = K / 128;
  if (split > groups) split = static_cast<int>(groups);
  if (split > 1 && (ws == nullptr || ws_bytes < static_cast<size_t>(split) * M * N * sizeof(float)))
    return BP_E_WORKSPACE;
  const int64_t tiles = (N + tile_rows - 1) / tile_rows;
  if (tiles > 0x7fffffff) return BP_E_INVALID_ARG;
  dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(split));
  if (mf_fn != nullptr) {
    const size_t lds = pro.kind != 0 ? static_cast<size_t>((2 * M + 2) * K * 2) : 0;
    mf_fn<<<grid, waves * kWave, lds, st>>>(static_cast<const uint16_t*>(x), static_cast<const uint8_t*>(packed),
                                            scale, scale_dt, static_cast<const uint16_t*>(zero),
                                            static_cast<uint16_t*>(y), static_cast<float*>(ws), static_cast<int>(M),
                                            N, K, split, pro);
  } else {
    fn<<<grid, waves * kWave, 0, st>>>(static_cast<const uint16_t*>(x), static_cast<const uint8_t*>(packed), scale,
                                       scale_dt, static_cast<const uint16_t*>(zero), static_cast<uint16_t*>(y),
                                       static_cast<float*>(ws), static_cast<int>(M), N, K, split);
  }
  const int rc = launch_status();
  if (rc != BP_OK || split == 1) return rc;
  splitk_reduce_kernel<<<grid_for(M * N), 256, 0, st>>>(static_cast<const float*>(ws), static_cast<uint16_t*>(y),
                                                       nullptr, 0, M, N, split);
  return launch_status();
}

}  // namespace

int splitk_reduce_launch(const float* ws, uint16_t* y, const void* scale, int scale_dt, int64_t M, int64_t N,
                         int split, hipStream_t st) {
  splitk_reduce_kernel<<<grid_for(M * N), 256, 0, st>>>(ws, y, scale, scale_dt, M, N, split);
  return launch_status();
}

}  // namespace bp

extern "C" {

int bp_skinny_int4_config_supported(int mt, int tile_rows, int waves) {
  return bp::int4_pick(mt, tile_rows, waves) != nullptr ? 1 : 0;
}

int bp_skinny_int4(const void* x, const void* packed, const void* scale, int scale_dtype, const void* zero, void* y,
                   int64_t M, int64_t N, int64_t K, int tile_rows, int waves, int split, void* workspace,
                   size_t workspace_bytes, void* stream) {
  return bp::skinny_int4_launch(x, packed, scale, scale_dtype, zero, y, M, N, K, tile_rows, waves, split, workspace,
                                workspace_bytes, stream);
}

int bp_skinny_int4_pro(const void* x, const void* packed, const void* scale, int scale_dtype, const void* zero, void* y,
                       int64_t M, int64_t N, int64_t K, int tile_rows, int waves, int epilogue,
                       const BpPrologue* prologue, void* stream) {
  if (prologue == nullptr || epilogue < 0 || epilogue > 1) return BP_E_INVALID_ARG;
  return bp::skinny_int4_launch(x, packed, scale, scale_dtype, zero, y, M, epilogue ? 2 * N : N, K, tile_rows, waves,
                                1, nullptr, 0, stream, epilogue, prologue);
}

int bp_skinny_int4_silu(const void* x, const void* packed, const void* scale, int scale_dtype, const void* zero,
                        void* out, int64_t M, int64_t ffn, int64_t K, int tile_rows, int waves, void* stream) {
  if (ffn < 0) return BP_E_INVALID_ARG;
  return bp::skinny_int4_launch(x, packed, scale, scale_dtype, zero, out, M, 2 * ffn, K, tile_rows, waves, 1, nullptr,
                                0, stream, 1);
}

int bp_version(void) { return 100; }

const char* bp_status_string(int status) {
  switch (status) {
    case BP_OK: return "success";
    case BP_E_INVALID_ARG: return "invalid argument (null pointer, negative size or inconsistent shape)";
    case BP_E_UNSUPPORTED: return "unsupported tile configuration or dtype";
    case BP_E_WORKSPACE: return "split-K workspace missing or too small";
    default: return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status)) : "unknown status";
  }
}

size_t bp_skinny_workspace_bytes(int64_t M, int64_t N, int split) {
  if (split <= 1 || M <= 0 || N <= 0) return 0;
  return static_cast<size_t>(split) * static_cast<size_t>(M) * static_cast<size_t>(N) * sizeof(float);
}

int bp_splitk_reduce(const void* workspace, void* y, const void* scale, int scale_dtype, int64_t M, int64_t N,
                     int split, void* stream) {
  if (M < 0 || N < 0 || split < 1) return BP_E_INVALID_ARG;
  if (M == 0 || N == 0) return BP_OK;
  if (workspace == nullptr || y == nullptr) return BP_E_INVALID_ARG;
  if (scale != nullptr && (scale_dtype < BP_DT_BF16 || scale_dtype > BP_DT_F32)) return BP_E_INVALID_ARG;
  bp::splitk_reduce_kernel<<<bp::grid_for(M * N), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const float*>(workspace), static_cast<uint16_t*>(y), scale, scale_dtype, M, N, split);
  return bp::launch_status();
}

}  // extern "C"
