// Signed activation FHT: y = (S H S pad(x))[:F] per row, S = diag(signs), H the
// normalized Sylvester Walsh-Hadamard transform of order P = 2^LB >= F.
//
// Reference: FixedFHTMix.forward (examples/nanogpt/model.py:200-218: pad the
// last dimension to P, multiply by the ±1 sign buffer, normalized_fht_last_dim
// (:180-197), multiply by the signs again, keep the first F).  S H S is
// symmetric, so the same kernel computes the backward on the gradient.
//
// One row per thread group of the whole-block VALU geometry (Geo<LB>), the
// workgroups looping over row groups.  A row stays in the coalesced layout
// (register r of thread t holds position r * TB + t), so it is loaded, signed
// (a per-thread sign mask read once per workgroup) and stored without staging,
// and the transform starts on the register bits and needs one LDS exchange per
// remaining 5-bit group plus one back.  Each thread reads its values before it
// writes any, and every position is read and written by the same thread, so
// the output may alias the input.
#include "bfht_device.h"
#include "bfht_launch.h"

namespace lwl {
namespace {

// Workgroups of one launch: each loops over row groups, so the sign mask is
// built once per workgroup.
constexpr int64_t kMixMaxGrid = 2048;

template <int LB, class T>
__global__ __launch_bounds__(Geo<LB>::WG) void bfht_mix_rows(const T* x, T* out, const float* __restrict__ signs,
                                                            int64_t rows, int features) {
  using Gm = Geo<LB>;
  __shared__ float smem[Gm::LDS_FLOATS];
  const int gi = threadIdx.x >> Gm::LT;
  const int t = threadIdx.x & (Gm::TB - 1);
  float* lds = smem + (Gm::NG > 1 ? gi * Gm::PADDED : 0);
  // coalesced layout: register r holds position r * TB + t (for TB = 1, the
  // whole row); bit r of the mask = sign of that position
  uint32_t neg = 0;
#pragma unroll
  for (int r = 0; r < Gm::E; ++r) neg |= (uint32_t)(signs[r * Gm::TB + t] < 0.0f) << r;
  auto flip = [&](float v, int r) { return __uint_as_float(__float_as_uint(v) ^ (((neg >> r) & 1u) << 31)); };
  const float scale = inv_sqrt_block<LB>();
  const int64_t groups = (rows + Gm::G - 1) / Gm::G;
  for (int64_t rg = blockIdx.x; rg < groups; rg += gridDim.x) {
    const int64_t row = rg * Gm::G + gi;
    const bool active = row < rows;
    const T* xr = x + (active ? row : 0) * features;
    T* orow = out + row * features;
    float v[Gm::E];
    // loads from a valid index (position 0 of the row stands in for the padding)
    // and a select, so all E loads are in flight at once
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) {
      const int p = r * Gm::TB + t;
      const bool ok = active && p < features;
      const float xv = to_f32(xr[ok ? p : 0]);
      v[r] = flip(ok ? xv : 0.0f, r);
    }
    fht_coalesced<LB, Gm::LE>(v, lds, t);
    if (active) {
#pragma unroll
      for (int r = 0; r < Gm::E; ++r) {
        const int p = r * Gm::TB + t;
        if (p < features) orow[p] = from_f32<T>(flip(v[r] * scale, r));
      }
    }
  }
}

template <int LB, class T>
hipError_t launch_mix_lb(const void* x, void* out, const float* signs, int64_t rows, int64_t features,
                         hipStream_t s) {
  using Gm = Geo<LB>;
  const int64_t groups = (rows + Gm::G - 1) / Gm::G;
  const int64_t grid = groups < kMixMaxGrid ? groups : kMixMaxGrid;
  hipLaunchKernelGGL((bfht_mix_rows<LB, T>), dim3((unsigned)grid), dim3(Gm::WG), 0, s, static_cast<const T*>(x),
                     static_cast<T*>(out), signs, rows, (int)features);
  return hipGetLastError();
}

template <class T, int... LBs>
hipError_t dispatch_mix(int LB, const void* x, void* out, const float* signs, int64_t rows, int64_t features,
                        hipStream_t s, std::integer_sequence<int, LBs...>) {
  using Fn = hipError_t (*)(const void*, void*, const float*, int64_t, int64_t, hipStream_t);
  static const Fn table[] = {&launch_mix_lb<LBs, T>...};
  return table[LB](x, out, signs, rows, features, s);
}

}  // namespace

hipError_t launch_fht_mix(int dtype, const void* x, void* out, const float* signs, int64_t rows, int64_t features,
                          int log_size, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  if (log_size < 0 || log_size > kTileLog) return hipErrorInvalidValue;
  const auto seq = std::make_integer_sequence<int, kTileLog + 1>{};
  switch (dtype) {
    case kF32: return dispatch_mix<float>(log_size, x, out, signs, rows, features, s, seq);
    case kF16: return dispatch_mix<f16>(log_size, x, out, signs, rows, features, s, seq);
    case kBF16: return dispatch_mix<bf16>(log_size, x, out, signs, rows, features, s, seq);
  }
  return hipErrorInvalidValue;
}

}  // namespace lwl
