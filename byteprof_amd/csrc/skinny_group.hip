// Grouped skinny launch: G independent linears at one activation row, y_g = x_g . W_g^T, in one non-persistent grid.
//
// Launched one at a time, a set of small linears is bound by the fixed cost of each launch and by the tail of each
// short weight stream (a 2048 x 2048 bf16 weight streams in ~1 us on MI355X, a dependent launch costs ~1.6 us). The
// grouped launch concatenates the row blocks of every linear into one grid: workgroup b takes ROWS consecutive rows
// of the item whose block range holds b, so the hardware dispatcher streams the whole set back to back with as many
// short-lived workgroups per CU as occupancy allows (no persistent waves, no cross-workgroup traffic).
//
// Work per workgroup is skinny_dot_kernel's at one activation row (skinny_kernel.h): chunk c of a row (1 KiB, 64
// lanes x 16 bytes) goes to wave c % WAVES, each lane accumulates v_dot2_f32_bf16 products in fp32, the wave sum is
// wave_transpose_reduce, the wave totals are added in LDS in wave order, the int8 scale multiplies the fp32 total
// and the result is rounded to nearest-even bf16. The same helpers in the same order make every output bitwise equal
// to skinny_mm's at the same (rows, waves) with split 1.
//
// Item lookup: items[i].block0 is the first workgroup of item i (ascending); lut[j] is the item holding workgroup
// j * kGroupLutSpan. A workgroup reads lut[b / span] and walks forward while the next item starts at or before b;
// the walk passes only items whose whole block range lies inside one lut span, i.e. items of fewer than span
// workgroups (none for the decode-step set at 2 rows per workgroup).
//
// Reference semantics: byteprof/optim/skinny.py:36-90 (_skinny_kernel at split 1), :136-166 (skinny_mm), run once
// per linear of the set by tools/skinny_bench.py:45-71.

#include "byteprof_amd.h"
#include "skinny_kernel.h"

namespace bp {
namespace {

constexpr int kGroupLutSpan = BP_GROUP_LUT_SPAN;

template <int KIND, int ROWS, int WAVES>
__global__ __launch_bounds__(WAVES * kWave) void skinny_group_kernel(const BpGroupItem* __restrict__ items,
                                                                     const int32_t* __restrict__ lut, int num_items,
                                                                     int scale_dt) {
  using L = Layout<KIND>;
  __shared__ float red[WAVES][ROWS];

  const int blk = static_cast<int>(blockIdx.x);
  int g = lut[blk / kGroupLutSpan];
  while (g + 1 < num_items && items[g + 1].block0 <= blk) ++g;
  const BpGroupItem it = items[g];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t N = it.N;
  const int64_t K = it.K;
  const int64_t row0 = static_cast<int64_t>(blk - it.block0) * ROWS;
  const int nch = static_cast<int>(K / L::kChunk);
  const uint8_t* __restrict__ w = static_cast<const uint8_t*>(it.w);
  const uint16_t* __restrict__ x = static_cast<const uint16_t*>(it.x);

  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) acc[r] = 0.f;

  for (int c = wave; c < nch; c += WAVES) {
    const int64_t k0 = static_cast<int64_t>(c) * L::kChunk + static_cast<int64_t>(lane) * L::kEpl;
    u32x4 wv[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      wv[r] = u32x4{0u, 0u, 0u, 0u};
      if (row0 + r < N) wv[r] = load_w<KIND, true>(w, row0 + r, K, k0);
    }
    uint32_t xv[L::kXDwords];
    load_x<KIND, true>(x, K, k0, xv);
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = chunk_dot<KIND>(wv[r], xv, acc[r]);
  }

  wave_transpose_reduce<ROWS>(acc, lane);
  // Lane l holds the wave total of row l / (64 / ROWS).
  if ((lane & (kWave / ROWS - 1)) == 0) red[wave][lane / (kWave / ROWS)] = acc[0];
  __syncthreads();

  if (threadIdx.x < ROWS) {
    const int64_t row = row0 + threadIdx.x;
    if (row < N) {
      float t = red[0][threadIdx.x];
#pragma unroll
      for (int v = 1; v < WAVES; ++v) t += red[v][threadIdx.x];
      if constexpr (KIND == kInt8) t *= load_scale(it.scale, row, scale_dt);
      static_cast<uint16_t*>(it.y)[row] = float_to_bf16_bits(t);
    }
  }
}

using GroupFn = void (*)(const BpGroupItem*, const int32_t*, int, int);

template <int KIND, int ROWS>
GroupFn pick_waves(int waves) {
  switch (waves) {
    case 1: return &skinny_group_kernel<KIND, ROWS, 1>;
    case 2: return &skinny_group_kernel<KIND, ROWS, 2>;
    case 4: return &skinny_group_kernel<KIND, ROWS, 4>;
    case 8: return &skinny_group_kernel<KIND, ROWS, 8>;
    default: return nullptr;
  }
}

template <int KIND>
GroupFn pick_rows(int rows, int waves) {
  switch (rows) {
    case 1: return pick_waves<KIND, 1>(waves);
    case 2: return pick_waves<KIND, 2>(waves);
    case 4: return pick_waves<KIND, 4>(waves);
    case 8: return pick_waves<KIND, 8>(waves);
    default: return nullptr;
  }
}

GroupFn group_pick(int wkind, int rows, int waves) {
  if (wkind == kBf16) return pick_rows<kBf16>(rows, waves);
  if (wkind == kInt8) return pick_rows<kInt8>(rows, waves);
  return nullptr;
}

int64_t group_chunk(int wkind) { return wkind == kBf16 ? Layout<kBf16>::kChunk : Layout<kInt8>::kChunk; }

int group_launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? BP_OK : static_cast<int>(e);
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Checks an item's operands (everything but block0); BP_OK or a BP_E_* code.
int check_item(const BpGroupItem& it, int wkind) {
  if (it.N < 0 || it.K <= 0 || it.K % group_chunk(wkind) != 0) return BP_E_INVALID_ARG;
  if (it.N == 0) return BP_OK;
  if (it.x == nullptr || it.w == nullptr || it.y == nullptr) return BP_E_INVALID_ARG;
  if (!aligned16(it.x) || !aligned16(it.w)) return BP_E_INVALID_ARG;
  if (wkind == kInt8 && it.scale == nullptr) return BP_E_INVALID_ARG;
  return BP_OK;
}

}  // namespace
}  // namespace bp

extern "C" {

int bp_skinny_group_config_supported(int wkind, int rows, int waves) {
  return bp::group_pick(wkind, rows, waves) != nullptr ? 1 : 0;
}

int bp_skinny_group_plan(BpGroupItem* items, int num_items, int wkind, int rows, int32_t* lut, int lut_capacity) {
  if (items == nullptr || num_items <= 0 || rows <= 0) return BP_E_INVALID_ARG;
  if (wkind != bp::kBf16 && wkind != bp::kInt8) return BP_E_UNSUPPORTED;
  int64_t blocks = 0;
  for (int i = 0; i < num_items; ++i) {
    const int rc = bp::check_item(items[i], wkind);
    if (rc != BP_OK) return rc;
    items[i].block0 = static_cast<int32_t>(blocks);
    blocks += (items[i].N + rows - 1) / rows;
    if (blocks > 0x7fffffff) return BP_E_INVALID_ARG;
  }
  if (lut != nullptr) {
    const int64_t spans = (blocks + bp::kGroupLutSpan - 1) / bp::kGroupLutSpan;
    if (spans > lut_capacity) return BP_E_INVALID_ARG;
    int g = 0;
    for (int64_t j = 0; j < spans; ++j) {
      const int64_t b = j * bp::kGroupLutSpan;
      while (g + 1 < num_items && items[g + 1].block0 <= b) ++g;
      lut[j] = g;
    }
  }
  return static_cast<int>(blocks);
}

int bp_skinny_group_run(int wkind, int scale_dtype, const BpGroupItem* host_items, const void* dev_items,
                        const void* dev_lut, int num_items, int blocks, int rows, int waves, void* stream) {
  if (host_items == nullptr || num_items <= 0 || blocks < 0) return BP_E_INVALID_ARG;
  bp::GroupFn fn = bp::group_pick(wkind, rows, waves);
  if (fn == nullptr) return BP_E_UNSUPPORTED;
  if (wkind == bp::kInt8 && (scale_dtype < BP_DT_BF16 || scale_dtype > BP_DT_F32)) return BP_E_INVALID_ARG;
  // The host copy must be the plan of these items at these rows: checked item by item.
  int64_t next = 0;
  for (int i = 0; i < num_items; ++i) {
    const BpGroupItem& it = host_items[i];
    const int rc = bp::check_item(it, wkind);
    if (rc != BP_OK) return rc;
    if (it.block0 != next) return BP_E_INVALID_ARG;
    next += (it.N + rows - 1) / rows;
  }
  if (next != blocks) return BP_E_INVALID_ARG;
  if (blocks == 0) return BP_OK;
  if (dev_items == nullptr || dev_lut == nullptr) return BP_E_INVALID_ARG;
  fn<<<blocks, waves * bp::kWave, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const BpGroupItem*>(dev_items), static_cast<const int32_t*>(dev_lut), num_items, scale_dtype);
  return bp::group_launch_status();
}

}  // extern "C"
