// Kernels and C ABI of the matrix-core skinny matmul with the 8-row segment layout (skinny_mf.h): the plain launch
// (any M up to 64, split-K through the fixed-order reduce), its gate|up + SiLU epilogue and its partial sums for a
// caller-side reduce.
//
// Reference semantics: byteprof/optim/skinny.py:36-90 (kernel and _split_reduce), :93-133 (_launch), via skinny_mm
// (skinny.py:136-166).

#include <algorithm>
#include <mutex>

#define BP_MF_INSTANTIATE
#include "skinny_mf_kernel.h"

namespace bp {

// Fixed-order split reduce of skinny.hip.
int splitk_reduce_launch(const float* ws, uint16_t* y, const void* scale, int scale_dt, int64_t M, int64_t N,
                         int split, hipStream_t st);

// Launches whose waves have 4, 8 or 16 segments each are instantiated in skinny_mf_n4 / n8 / n16.hip.
extern template MfFn mf_pick_n<4>(int, int, int, int, bool, int, bool, bool, int);
extern template MfFn mf_pick_n<8>(int, int, int, int, bool, int, bool, bool, int);
extern template MfFn mf_pick_n<16>(int, int, int, int, bool, int, bool, bool, int);
template MfFn mf_pick_n<0>(int, int, int, int, bool, int, bool, bool, int);

namespace {

// The kernel of a launch: the straight-line variant when every wave has exactly 4, 8 or 16 segments (nseg_wave),
// else the general one.
MfFn mf_pick(int wkind, int mb, int rb, int waves, bool vec, int epi, bool xl, bool pro = false, int nseg_wave = 0,
             int wr = 1) {
  switch (vec ? nseg_wave : 0) {
    case 4: return mf_pick_n<4>(wkind, mb, rb, waves, vec, epi, xl, pro, wr);
    case 8: return mf_pick_n<8>(wkind, mb, rb, waves, vec, epi, xl, pro, wr);
    case 16: return mf_pick_n<16>(wkind, mb, rb, waves, vec, epi, xl, pro, wr);
    default: return mf_pick_n<0>(wkind, mb, rb, waves, vec, epi, xl, pro, wr);
  }
}

// Row groups of a launch's xstage flags (BP_XS_ROWS2 / BP_XS_ROWS4, with BP_XS_STAGE), 1 without.
int mf_row_groups(int xstage) {
  if (!(xstage & BP_XS_STAGE)) return 1;
  return (xstage & BP_XS_ROWS4) ? 4 : (xstage & BP_XS_ROWS2) ? 2 : 1;
}

int mf_blocks(int64_t M) { return M <= 8 ? 1 : M <= 16 ? 2 : M <= 32 ? 4 : 8; }

int mf_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}

__global__ void mf_fill_zero_kernel(uint16_t* __restrict__ y, int64_t count) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    y[i] = 0;
}

#ifdef BP_TIMELINE
// Timeline builds: the stamps of the last launch's workgroups (MfPro::tl), read by bp_mf_timeline_read.
__device__ unsigned long long mf_timeline[kMfTimelineWgs * 8];

unsigned long long* mf_timeline_buffer() {
  void* p = nullptr;
  return hipGetSymbolAddress(&p, HIP_SYMBOL(mf_timeline)) == hipSuccess ? static_cast<unsigned long long*>(p)
                                                                          : nullptr;
}
#endif

constexpr int64_t kMaxStageBytes = 32 * 1024;  // LDS for staged activations (dynamic shared memory)
constexpr int64_t kMaxStageBytesRows = 64 * 1024;  // with row groups (one copy serves 2-4x the rows)
constexpr int64_t kMaxProLdsBytes = 80 * 1024;  // with a norm prologue's gamma and residual rows as well

// LDS bytes of the staged activations of a launch (the largest K range of a workgroup), or -1 when they do not fit
// (limit: kMaxStageBytes, with row groups kMaxStageBytesRows).
int64_t mf_stage_bytes(int wkind, int64_t M, int64_t K, int split, int wr = 1) {
  const int64_t seg = wkind == kBf16 ? 64 : 128;
  const int64_t nseg = (K + seg - 1) / seg;
  const int64_t per = (nseg + split - 1) / split;
  const int64_t rows = M < 8 * mf_blocks(M) ? M : 8 * mf_blocks(M);
  const int64_t bytes = rows * per * seg * 2;
  return bytes <= (wr > 1 ? kMaxStageBytesRows : kMaxStageBytes) ? bytes : -1;
}

constexpr int64_t kMaxVecK = int64_t{1} << 24;  // 2 x 64 rows x K bytes of activations < 2^31

// mode 0: y (split > 1: partials then the reduce); 1: partials only (split >= 2, y unused); 2: SiLU epilogue.
int mf_launch(int wkind, const void* x, const void* w, const void* scale, int scale_dt, void* y, int64_t M,
              int64_t N, int64_t K, int rb, int waves, int split, int xstage, void* ws, size_t ws_bytes, void* stream,
              int mode, const BpPrologue* prologue = nullptr) {
  if (wkind != kBf16 && wkind != kInt8) return BP_E_UNSUPPORTED;
  if (M < 0 || N < 0 || K < 0 || M > 64) return BP_E_INVALID_ARG;
  if (M == 0 || N == 0) return BP_OK;
  if (x == nullptr || w == nullptr || (mode != 1 && y == nullptr)) return BP_E_INVALID_ARG;
  if (wkind == kInt8 && mode != 1 && (scale == nullptr || scale_dt < BP_DT_BF16 || scale_dt > BP_DT_F32))
    return BP_E_INVALID_ARG;
  if (split < 1 || split > 1024) return BP_E_UNSUPPORTED;
  if (mode == 2 && (N % 2 != 0 || split != 1 || M > 16)) return BP_E_UNSUPPORTED;
  if (mode == 1 && split < 2) return BP_E_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (K == 0) {
    if (mode == 1) return BP_E_UNSUPPORTED;
    const int64_t count = mode == 2 ? M * (N / 2) : M * N;
    mf_fill_zero_kernel<<<static_cast<unsigned>(std::min<int64_t>((count + 255) / 256, 2048)), 256, 0, st>>>(
        static_cast<uint16_t*>(y), count);
    return mf_status();
  }
  // xstage bit 1: the general segment loop even where the straight-line kernel of the count applies
  const bool general = (xstage & BP_XS_GENERAL) != 0;
  int wr = mf_row_groups(xstage);
  xstage &= BP_XS_STAGE;
  const int64_t seg = wkind == kBf16 ? 64 : 128;
  // the vector loads read whole segments: K a multiple of the segment, 16-byte aligned operands, and K below
  // 2^24, so that up to 64 activation rows lie within one buffer resource (2 M K < 2^31 bytes) whatever M is: the
  // choice, and with it the K order, does not depend on M
  const bool vec = K % seg == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(w) % 16 == 0 && K < kMaxVecK;
  if (!vec) {
    rb = 1;
    waves = 4;
    xstage = 0;
    wr = 1;
  }
  const int64_t nseg = (K + seg - 1) / seg;
  if (split > nseg) split = static_cast<int>(nseg);
  if (mode == 1 && split < 2) return BP_E_UNSUPPORTED;
  MfPro pro{0, 0.f, nullptr, nullptr, nullptr, 0, nullptr};
  if (prologue != nullptr && prologue->kind != 0) {
    // whole rows staged in LDS: split 1, vector loads, at most 16 rows
    if (prologue->kind != BP_PRO_UNIT_RMS && prologue->kind != BP_PRO_NORM) return BP_E_INVALID_ARG;
    if (prologue->kind == BP_PRO_NORM && prologue->gamma == nullptr) return BP_E_INVALID_ARG;
    // gamma, the residual and xout are read / written in 16-byte pieces
    if (reinterpret_cast<uintptr_t>(prologue->gamma) % 16 != 0 || reinterpret_cast<uintptr_t>(prologue->residual) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(prologue->xout) % 16 != 0 || reinterpret_cast<uintptr_t>(prologue->gamma2) % 16 != 0)
      return BP_E_INVALID_ARG;
    if (prologue->gamma2 != nullptr && prologue->kind != BP_PRO_NORM) return BP_E_INVALID_ARG;
    // workgroup (0, 0) writes xout while the others still read x and the residual rows
    const int64_t rows_bytes = 2 * M * K;
    if (ranges_overlap(prologue->xout, rows_bytes, x, rows_bytes) ||
        (prologue->kind == BP_PRO_NORM && ranges_overlap(prologue->xout, rows_bytes, prologue->residual, rows_bytes)))
      return BP_E_INVALID_ARG;
    if (!vec || split != 1 || M > 16 || mode == 1) return BP_E_UNSUPPORTED;
    xstage = 1;
    wr = 1;
    pro = MfPro{prologue->kind, prologue->eps, static_cast<const uint16_t*>(prologue->gamma),
                static_cast<const uint16_t*>(prologue->residual), static_cast<uint16_t*>(prologue->xout), 0,
                static_cast<const uint16_t*>(prologue->gamma2)};
  }
  int64_t lds = 0;
  if (xstage) {
    lds = mf_stage_bytes(wkind, M, K, split, wr);
    if (lds < 0) return BP_E_UNSUPPORTED;
  }
  if (pro.kind == BP_PRO_NORM) {
    // gamma and the residual rows staged in LDS after the rows (mf_prologue reads them from there), when they fit;
    // otherwise the prologue reads them from memory
    const int64_t gl = 2 * K * (1 + (pro.residual != nullptr ? M : 0) + (pro.gamma2 != nullptr ? 1 : 0));
    if (M == 1 || lds + gl <= kMaxProLdsBytes) {
      pro.gl = 1;
      lds += gl;
    }
  }
#ifdef BP_TIMELINE
  pro.tl = mf_timeline_buffer();
#endif
  // every wave has the same segment count when the split ranges and the waves divide the segments evenly
  int nseg_wave = !general && nseg % split == 0 && (nseg / split) % waves == 0
                      ? static_cast<int>(nseg / split / waves)
                      : 0;
  if (wr > 1 && nseg_wave == 16) nseg_wave = 0;  // the row-group kernels run the general loop there
  MfFn fn = mf_pick(wkind, mf_blocks(M), rb, waves, vec, mode == 2 ? 1 : 0, xstage != 0, pro.kind != 0, nseg_wave,
                    wr);
  if (fn == nullptr && wr == 4) {
    // row groups are a plan, not a K order: without a compiled kernel of 4 groups, 2 (the same LDS)
    wr = 2;
    fn = mf_pick(wkind, mf_blocks(M), rb, waves, vec, mode == 2 ? 1 : 0, xstage != 0, pro.kind != 0, nseg_wave, wr);
  }
  if (fn == nullptr && wr > 1 && pro.kind == 0) {
    // without a row-group kernel (rows outside 9..16, rb or waves outside its menu), the same sums from one group,
    // staged where the rows fit in the plain limit
    wr = 1;
    if (xstage) {
      lds = mf_stage_bytes(wkind, M, K, split, 1);
      if (lds < 0) {
        xstage = 0;
        lds = 0;
      }
    }
    fn = mf_pick(wkind, mf_blocks(M), rb, waves, vec, mode == 2 ? 1 : 0, xstage != 0, false, nseg_wave);
  }
  if (fn == nullptr) return BP_E_UNSUPPORTED;
  if (split > 1 && (ws == nullptr || ws_bytes < static_cast<size_t>(split) * M * N * sizeof(float)))
    return BP_E_WORKSPACE;
  const int64_t tiles = (N + 8 * rb * wr - 1) / (8 * rb * wr);
  if (tiles > 0x7fffffff) return BP_E_INVALID_ARG;
  fn<<<dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(split)), waves * wr * kWave, static_cast<size_t>(lds),
       st>>>(static_cast<const uint16_t*>(x), static_cast<const uint8_t*>(w), scale, scale_dt,
             static_cast<uint16_t*>(y), static_cast<float*>(ws), static_cast<int>(M), N, K, split, pro);
  const int rc = mf_status();
  if (rc != BP_OK || split == 1 || mode == 1) return rc;
  return splitk_reduce_launch(static_cast<const float*>(ws), static_cast<uint16_t*>(y),
                              wkind == kInt8 ? scale : nullptr, scale_dt, M, N, split, st);
}

// The split-K partials of bp_skinny_mf_static: a fixed device array instead of a caller's workspace. Each GPU the
// library runs on holds its own copy until the process ends; host code uses the per-device address from
// hipGetSymbolAddress (static_scratch), never the array's name.
constexpr size_t kStaticScratchBytes = size_t{8} << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;

// The device address of `scratch` on the current device (resolved once per device), or null on error.
void* static_scratch() {
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

}  // namespace
}  // namespace bp

extern "C" {

#ifdef BP_TIMELINE
// Timeline builds only: the per-workgroup stamps of the last matrix-core launch, [16384][8] uint64.
int bp_mf_timeline_read(void* dst, size_t bytes) {
  if (dst == nullptr || bytes < sizeof(unsigned long long) * bp::kMfTimelineWgs * 8) return BP_E_INVALID_ARG;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(bp::mf_timeline), sizeof(unsigned long long) * bp::kMfTimelineWgs * 8) ==
                 hipSuccess
             ? BP_OK
             : BP_E_INVALID_ARG;
}
#endif

size_t bp_skinny_mf_static_bytes(void) { return bp::kStaticScratchBytes; }

int bp_skinny_mf_static(int wkind, const void* x, const void* w, const void* scale, int scale_dtype, void* y,
                        int64_t M, int64_t N, int64_t K, int rb, int waves, int split, int xstage, void* stream) {
  if (M < 0 || N < 0 || split < 1) return BP_E_INVALID_ARG;
  if (split > 1 && M > 0 && N > 0 &&
      static_cast<double>(split) * static_cast<double>(M) * static_cast<double>(N) * sizeof(float) >
          static_cast<double>(bp::kStaticScratchBytes))
    return BP_E_WORKSPACE;
  void* ws = nullptr;
  if (split > 1) {
    ws = bp::static_scratch();
    if (ws == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
  }
  return bp::mf_launch(wkind, x, w, scale, scale_dtype, y, M, N, K, rb, waves, split, xstage, ws,
                       split > 1 ? bp::kStaticScratchBytes : 0, stream, 0);
}

int bp_skinny_mf_supported(int wkind, int M, int rb, int waves, int xstage) {
  if (M < 1 || M > 64) return 0;
  const int wr = bp::mf_row_groups(xstage);
  // the row-group kernels exist for the straight-line counts 4 and 8 and the general loop; report the general one
  return bp::mf_pick(wkind, bp::mf_blocks(M), rb, waves, true, 0, (xstage & BP_XS_STAGE) != 0, false, 0, wr) !=
                 nullptr
             ? 1
             : 0;
}

int bp_skinny_mf_k_segment(int wkind) { return wkind == bp::kBf16 ? 64 : wkind == bp::kInt8 ? 128 : 0; }

int64_t bp_skinny_mf_stage_bytes(int wkind, int64_t M, int64_t K, int split) {
  if ((wkind != bp::kBf16 && wkind != bp::kInt8) || M < 1 || M > 64 || K < 1 || split < 1) return -1;
  return bp::mf_stage_bytes(wkind, M, K, split);
}

int64_t bp_skinny_mf_stage_bytes_rows(int wkind, int64_t M, int64_t K, int split, int xstage) {
  if ((wkind != bp::kBf16 && wkind != bp::kInt8) || M < 1 || M > 64 || K < 1 || split < 1) return -1;
  return bp::mf_stage_bytes(wkind, M, K, split, bp::mf_row_groups(xstage | BP_XS_STAGE));
}

int bp_skinny_mf(int wkind, const void* x, const void* w, const void* scale, int scale_dtype, void* y, int64_t M,
                 int64_t N, int64_t K, int rb, int waves, int split, int xstage, void* workspace,
                 size_t workspace_bytes, void* stream) {
  return bp::mf_launch(wkind, x, w, scale, scale_dtype, y, M, N, K, rb, waves, split, xstage, workspace,
                       workspace_bytes, stream, 0);
}

int bp_skinny_mf_partials(int wkind, const void* x, const void* w, int64_t M, int64_t N, int64_t K, int rb,
                          int waves, int split, int xstage, void* workspace, size_t workspace_bytes, void* stream) {
  if (workspace == nullptr) return BP_E_WORKSPACE;
  return bp::mf_launch(wkind, x, w, nullptr, 0, nullptr, M, N, K, rb, waves, split, xstage, workspace,
                       workspace_bytes, stream, 1);
}

int bp_skinny_mf_pro(int wkind, const void* x, const void* w, const void* scale, int scale_dtype, void* y, int64_t M,
                     int64_t N, int64_t K, int rb, int waves, int epilogue, const BpPrologue* prologue, void* stream) {
  if (prologue == nullptr || (epilogue != 0 && epilogue != 1)) return BP_E_INVALID_ARG;
  if (epilogue == 1 && N < 0) return BP_E_INVALID_ARG;
  return bp::mf_launch(wkind, x, w, scale, scale_dtype, y, M, epilogue == 1 ? 2 * N : N, K, rb, waves, 1, 1, nullptr,
                       0, stream, epilogue == 1 ? 2 : 0, prologue);
}

int bp_skinny_mf_silu(int wkind, const void* x, const void* w, const void* scale, int scale_dtype, void* out,
                      int64_t M, int64_t ffn, int64_t K, int rb, int waves, int xstage, void* stream) {
  if (ffn < 0) return BP_E_INVALID_ARG;
  return bp::mf_launch(wkind, x, w, scale, scale_dtype, out, M, 2 * ffn, K, rb, waves, 1, xstage, nullptr, 0, stream,
                       2);
}

}  // extern "C"
