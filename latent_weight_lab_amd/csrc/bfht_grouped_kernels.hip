// Grouped weight-cache kernels on the whole-block VALU transform: the slots of
// several generators (jobs) in one grid, each workgroup serving one job (the
// table's prefix sums count workgroups), each block running the code of its
// per-generator launch with the cache epilogue folded into its stores (forward)
// or the weight gradient's cast folded into its loads (backward).  The latent
// dtype T and the weight dtype W are template parameters, so the element
// accesses are straight typed loads and stores.
//
// Reference: latent_weight_lab/block_fht.py:503-569 (materialize_weight_cache,
// flush_weight_cache_to_latent_grad and the prepare / flush loops).
#include "bfht_block.h"

namespace lwl {
namespace {

// Store: the generator value rounded to T, times the weight scale rounded to T
// again (torch's `generator() * weight_scale` in T), then cast to W.
template <class T, class W>
struct WeightStore {
  W* out;
  float scale;
  __device__ __amdgpu_buffer_rsrc_t range(int64_t first, int64_t count) const {
    return tile_rsrc(out + first, (uint64_t)count * sizeof(W));
  }
  __device__ void operator()(__amdgpu_buffer_rsrc_t r, int i, float v) const { buf_store<W>(value(v), r, i); }
  __device__ void whole(__amdgpu_buffer_rsrc_t r, int base, int c, float v) const {
    buf_store_at<W>(value(v), r, base, c);
  }
  __device__ void at(int64_t i, float v) const { out[i] = from_f32<W>(value(v)); }
  __device__ float value(float v) const { return round_to<T>(round_to<T>(v) * scale); }
};

// Load: the weight gradient cast to T (torch's `grad.to(latent.dtype)`).
template <class T, class W>
struct WeightGradLoad {
  const W* g;
  __device__ __amdgpu_buffer_rsrc_t range(int64_t first, int64_t count) const {
    return tile_rsrc(g + first, (uint64_t)count * sizeof(W));
  }
  __device__ float operator()(__amdgpu_buffer_rsrc_t r, int i) const { return round_to<T>(buf_load<W>(r, i)); }
  __device__ float whole(__amdgpu_buffer_rsrc_t r, int base, int c) const {
    return round_to<T>(buf_load_at<W>(r, base, c));
  }
  __device__ float at(int64_t i) const { return round_to<T>(to_f32(g[i])); }
};

template <int LB, class T, class W>
__global__ __launch_bounds__(Geo<LB>::WG) void bfht_block_fwd_grouped(const GroupTable g) {
  __shared__ float smem[BlockLds<LB>::FLOATS];
  const int j = group_job(g, (int)blockIdx.x);
  const GroupJob& jb = g.job[j];
  const int64_t slot = (int64_t)(blockIdx.x - g.prefix[j]) * Geo<LB>::G + (threadIdx.x >> Geo<LB>::LT);
  block_fwd_slot<LB, T>(static_cast<const T*>(jb.src), WeightStore<T, W>{static_cast<W*>(jb.dst), jb.scale}, jb.n,
                        0, slot, jb.nblocks, 0, jb.size, jb.seed32, jb.layers, smem);
}

template <int LB, class T, class W>
__global__ __launch_bounds__(Geo<LB>::WG) void bfht_block_bwd_grouped(const GroupTable g) {
  __shared__ float smem[BlockLds<LB>::FLOATS];
  const int j = group_job(g, (int)blockIdx.x);
  const GroupJob& jb = g.job[j];
  const int64_t slot = (int64_t)(blockIdx.x - g.prefix[j]) * Geo<LB>::G + (threadIdx.x >> Geo<LB>::LT);
  block_bwd_slot<LB, T>(WeightGradLoad<T, W>{static_cast<const W*>(jb.src)}, static_cast<float*>(jb.part), jb.stride,
                        static_cast<T*>(nullptr), jb.n, 0, slot, jb.nblocks, 0, jb.size, jb.seed32, jb.layers, 0,
                        smem);
}

template <int LB, class T, class W>
hipError_t launch_lb(const GroupTable& g, hipStream_t s, bool fwd) {
  if (group_slots_per_wg(LB) != Geo<LB>::G) return hipErrorInvalidValue;  // the planner's prefix unit
  const dim3 grid((unsigned)g.prefix[g.count]), block(Geo<LB>::WG);
  if (fwd)
    hipLaunchKernelGGL((bfht_block_fwd_grouped<LB, T, W>), grid, block, 0, s, g);
  else
    hipLaunchKernelGGL((bfht_block_bwd_grouped<LB, T, W>), grid, block, 0, s, g);
  return hipGetLastError();
}

template <class T, class W, int... LBs>
hipError_t dispatch_lb(const GroupTable& g, int LB, hipStream_t s, bool fwd, std::integer_sequence<int, LBs...>) {
  using Fn = hipError_t (*)(const GroupTable&, hipStream_t, bool);
  static const Fn table[] = {&launch_lb<LBs, T, W>...};
  return table[LB](g, s, fwd);
}

template <class T>
hipError_t dispatch_w(const GroupTable& g, int wdtype, int LB, hipStream_t s, bool fwd) {
  const auto seq = std::make_integer_sequence<int, kTileLog + 1>{};
  switch (wdtype) {
    case kF32: return dispatch_lb<T, float>(g, LB, s, fwd, seq);
    case kF16: return dispatch_lb<T, f16>(g, LB, s, fwd, seq);
    case kBF16: return dispatch_lb<T, bf16>(g, LB, s, fwd, seq);
  }
  return hipErrorInvalidValue;
}

}  // namespace

int group_slots_per_wg(int log_block) {
  // Geo<LB>::G: blocks of 2^LB that one workgroup transforms together
  const int tb = 1 << (log_block - (log_block < 5 ? log_block : 5));
  return (tb < 256 ? 256 : tb) / tb;
}

hipError_t launch_block_grouped(const GroupTable& g, int dtype, int wdtype, int log_block, hipStream_t s,
                                bool fwd) {
  if (g.count <= 0 || g.prefix[g.count] == 0) return hipSuccess;
  if (log_block < 0 || log_block > kTileLog) return hipErrorInvalidValue;
  switch (dtype) {
    case kF32: return dispatch_w<float>(g, wdtype, log_block, s, fwd);
    case kF16: return dispatch_w<f16>(g, wdtype, log_block, s, fwd);
    case kBF16: return dispatch_w<bf16>(g, wdtype, log_block, s, fwd);
  }
  return hipErrorInvalidValue;
}

}  // namespace lwl
