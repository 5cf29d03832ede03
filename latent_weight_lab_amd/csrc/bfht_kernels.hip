// BlockFHT generation kernels for gfx950.
//
// Two families:
//  * whole-block kernels (B <= 2^15): one block per workgroup slot, resident
//    in VGPRs (32 per thread) with LDS exchanges, all layers in one launch;
//    small blocks pack several per workgroup.  Forward writes the requested
//    slice directly; backward writes one float32 partial per block (or the
//    final gradient when a single block is involved).
//  * tile passes (2^16 <= B <= 2^23): the block lives in a float32 work buffer
//    and each layer is two passes over 2^15-element LDS tiles — "low" transforms
//    index bits 0..14 of a contiguous chunk, "high" transforms bits 15..log2(B)-1
//    of a tile of 2^(log2B-15) rows x 2^(30-log2B) columns — so a layer costs two
//    reads and two writes of the work buffer instead of one per stage.  Signs,
//    the 1/sqrt(B) scale, zero padding, slicing and the latent/grad sources are
//    fused into the passes' loads and stores.
//
// Reference semantics: latent_weight_lab/block_fht.py:84-109 (forward),
// csrc/block_fht_ext_cuda.cu:185-223 and :568-622 (backward).
#include "bfht_device.h"
#include "bfht_launch.h"

namespace lwl {

template <int LB>
struct Geo {
  static constexpr int LE = LB < 5 ? LB : 5;  // log2 elements per thread
  static constexpr int E = 1 << LE;
  static constexpr int LT = LB - LE;          // log2 threads per block
  static constexpr int TB = 1 << LT;
  static constexpr int WG = TB < 256 ? 256 : TB;
  static constexpr int G = WG / TB;           // blocks per workgroup
  static constexpr int B = 1 << LB;
  static constexpr int NG = (LB + 4) / 5;
  static constexpr int PADDED = B + (B >> 5);
  static constexpr int LDS_FLOATS = NG > 1 ? G * PADDED : 1;
};

template <int LB>
__device__ __forceinline__ float inv_sqrt_block() {
  // 2^(-LB/2), exact for even LB
  return (LB & 1) ? 0.70710678118654752440f / (float)(1 << (LB >> 1)) : 1.0f / (float)(1 << (LB >> 1));
}

// ---------------------------------------------------------------- whole block

template <int LB, class T>
__global__ __launch_bounds__(Geo<LB>::WG) void bfht_block_fwd(const T* __restrict__ latent,
                                                             T* __restrict__ out, int n,
                                                             int64_t first_block, int64_t nblocks,
                                                             int64_t start, int64_t stop,
                                                             uint32_t seed32, int layers) {
  using Gm = Geo<LB>;
  __shared__ float smem[Gm::LDS_FLOATS];
  const int gi = threadIdx.x >> Gm::LT;
  const int t = threadIdx.x & (Gm::TB - 1);
  const int64_t slot = (int64_t)blockIdx.x * Gm::G + gi;
  const bool active = slot < nblocks;
  const int64_t block = first_block + (active ? slot : 0);
  float* lds = smem + (Gm::NG > 1 ? gi * Gm::PADDED : 0);
  const uint32_t bkey = block_key(seed32, block);
  const int p0 = t * Gm::E;
  const uint32_t word = (uint32_t)(p0 >> 5);

  float v[Gm::E];
  {
    const uint32_t w = sign_word(bkey, layer_key(0), word);
    if constexpr (Gm::NG > 1) {
      // coalesced: thread t loads positions k * TB + t, then takes its
      // contiguous run from the (padded, conflict-free) LDS copy
#pragma unroll
      for (int k = 0; k < Gm::E; ++k) {
        const int p = k * Gm::TB + t;
        lds[lds_index(p)] = p < n ? to_f32(latent[p]) : 0.0f;
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < Gm::E; ++r) v[r] = signed_by(lds[lds_index(p0 + r)], w, (p0 + r) & 31);
    } else {
#pragma unroll
      for (int r = 0; r < Gm::E; ++r) {
        const int p = p0 + r;
        const float x = p < n ? to_f32(latent[p]) : 0.0f;
        v[r] = signed_by(x, w, p & 31);
      }
    }
  }
  const float scale = inv_sqrt_block<LB>();
  for (int layer = 0; layer < layers; ++layer) {
    fht_unnormalized<LB, Gm::LE>(v, lds, t);
    const uint32_t w = sign_word(bkey, layer_key(layer + 1), word);
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) v[r] = signed_by(v[r], w, (p0 + r) & 31) * scale;
  }
  const int64_t base = block * Gm::B;
  const int64_t lo = start - base > 0 ? start - base : 0;
  const int64_t hi = stop - base < Gm::B ? stop - base : Gm::B;
  if constexpr (Gm::NG > 1) {
    // back through the LDS, so that consecutive threads store consecutive positions
    __syncthreads();  // the transform's last LDS reads are done
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) lds[lds_index(p0 + r)] = v[r];
    __syncthreads();
    if (!active) return;
#pragma unroll
    for (int k = 0; k < Gm::E; ++k) {
      const int p = k * Gm::TB + t;
      if (p >= lo && p < hi) out[base + p - start] = from_f32<T>(lds[lds_index(p)]);
    }
  } else {
    if (!active) return;
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) {
      const int p = p0 + r;
      if (p >= lo && p < hi) out[base + p - start] = from_f32<T>(v[r]);
    }
  }
}

// Backward: adjoint chain D_0 H D_1 ... H D_L on grad scattered into the block
// frame.  Writes partial[slot * n + p] (float32) for p < n, or the final
// gradient in T when `direct` (a single block).
template <int LB, class T>
__global__ __launch_bounds__(Geo<LB>::WG) void bfht_block_bwd(const T* __restrict__ grad,
                                                             float* __restrict__ partial,
                                                             T* __restrict__ grad_latent, int n,
                                                             int64_t first_block, int64_t nblocks,
                                                             int64_t start, int64_t stop,
                                                             uint32_t seed32, int layers,
                                                             int direct) {
  using Gm = Geo<LB>;
  __shared__ float smem[Gm::LDS_FLOATS];
  const int gi = threadIdx.x >> Gm::LT;
  const int t = threadIdx.x & (Gm::TB - 1);
  const int64_t slot = (int64_t)blockIdx.x * Gm::G + gi;
  const bool active = slot < nblocks;
  const int64_t block = first_block + (active ? slot : 0);
  float* lds = smem + (Gm::NG > 1 ? gi * Gm::PADDED : 0);
  const uint32_t bkey = block_key(seed32, block);
  const int p0 = t * Gm::E;
  const uint32_t word = (uint32_t)(p0 >> 5);
  const int64_t base = block * Gm::B;
  const int64_t lo = start - base > 0 ? start - base : 0;
  const int64_t hi = stop - base < Gm::B ? stop - base : Gm::B;

  float v[Gm::E];
  if constexpr (Gm::NG > 1) {
    // coalesced loads through the LDS (see bfht_block_fwd)
#pragma unroll
    for (int k = 0; k < Gm::E; ++k) {
      const int p = k * Gm::TB + t;
      lds[lds_index(p)] = (active && p >= lo && p < hi) ? to_f32(grad[base + p - start]) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) v[r] = lds[lds_index(p0 + r)];
  } else {
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) {
      const int p = p0 + r;
      v[r] = (active && p >= lo && p < hi) ? to_f32(grad[base + p - start]) : 0.0f;
    }
  }
  const float scale = inv_sqrt_block<LB>();
  for (int layer = layers - 1; layer >= 0; --layer) {
    const uint32_t w = sign_word(bkey, layer_key(layer + 1), word);
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) v[r] = signed_by(v[r], w, (p0 + r) & 31);
    fht_unnormalized<LB, Gm::LE>(v, lds, t);
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) v[r] *= scale;
  }
  const uint32_t w0 = sign_word(bkey, layer_key(0), word);
  if constexpr (Gm::NG > 1) {
    __syncthreads();  // the transform's last LDS reads are done
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) lds[lds_index(p0 + r)] = signed_by(v[r], w0, (p0 + r) & 31);
    __syncthreads();
    if (!active) return;
#pragma unroll
    for (int k = 0; k < Gm::E; ++k) {
      const int p = k * Gm::TB + t;
      if (p < n) {
        const float g = lds[lds_index(p)];
        if (direct)
          grad_latent[p] = from_f32<T>(g);
        else
          partial[slot * (int64_t)n + p] = g;
      }
    }
  } else {
    if (!active) return;
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) {
      const int p = p0 + r;
      if (p < n) {
        const float g = signed_by(v[r], w0, p & 31);
        if (direct)
          grad_latent[p] = from_f32<T>(g);
        else
          partial[slot * (int64_t)n + p] = g;
      }
    }
  }
}

// grad_latent[p] = sum_b part[b * stride + p], blocks in order.
// Fixed-order sum of the per-block float32 partial rows: grad[p] = sum over b
// of part[b * stride + p].  Each workgroup owns 128 columns (2 per lane); wave
// w adds rows w, w + 8, w + 16, ... in ascending order with 16 row loads in
// flight, and wave 0 adds the 8 wave sums in wave order, so the result does
// not depend on timing.  (A single column walk per thread keeps only a few
// loads in flight and leaves most of the chip idle for latent lengths of a
// few 10^4.)
constexpr int kRedWaves = 8;
constexpr int kRedCols = 128;
constexpr int kRedDepth = 16;

template <class T, bool kPairs>
__global__ __launch_bounds__(64 * kRedWaves) void bfht_reduce_blocks(const float* __restrict__ part,
                                                                     int64_t nblocks, int64_t stride, int n,
                                                                     T* __restrict__ grad_latent) {
  __shared__ float sums[kRedWaves][2][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c0 = blockIdx.x * kRedCols + 2 * lane;
  const bool has0 = c0 < n, has1 = c0 + 1 < n;
  float a0 = 0.0f, a1 = 0.0f;
  auto row = [&](int64_t b) -> float2 {
    const float* r = part + b * stride + c0;
    if (kPairs && has1) return *reinterpret_cast<const float2*>(r);
    return float2{has0 ? r[0] : 0.0f, has1 ? r[1] : 0.0f};
  };
  int64_t b = wave;
  for (; b + (int64_t)kRedWaves * (kRedDepth - 1) < nblocks; b += (int64_t)kRedWaves * kRedDepth) {
    float2 v[kRedDepth];
#pragma unroll
    for (int j = 0; j < kRedDepth; ++j) v[j] = row(b + (int64_t)kRedWaves * j);
#pragma unroll
    for (int j = 0; j < kRedDepth; ++j) {
      a0 += v[j].x;
      a1 += v[j].y;
    }
  }
  for (; b < nblocks; b += kRedWaves) {
    const float2 v = row(b);
    a0 += v.x;
    a1 += v.y;
  }
  sums[wave][0][lane] = a0;
  sums[wave][1][lane] = a1;
  __syncthreads();
  if (wave != 0) return;
  float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
  for (int w = 0; w < kRedWaves; ++w) {
    t0 += sums[w][0][lane];
    t1 += sums[w][1][lane];
  }
  if (has0) grad_latent[c0] = from_f32<T>(t0);
  if (has1) grad_latent[c0 + 1] = from_f32<T>(t1);
}

template <class T>
static hipError_t launch_reduce(const float* part, int64_t nblocks, int64_t stride, int64_t n, T* dst,
                                hipStream_t s) {
  const dim3 grid((unsigned)((n + kRedCols - 1) / kRedCols)), block(64 * kRedWaves);
  // 8-byte row loads need even column offsets in every row: part is 256-byte aligned
  if (stride % 2 == 0)
    hipLaunchKernelGGL((bfht_reduce_blocks<T, true>), grid, block, 0, s, part, nblocks, stride, (int)n, dst);
  else
    hipLaunchKernelGGL((bfht_reduce_blocks<T, false>), grid, block, 0, s, part, nblocks, stride, (int)n, dst);
  return hipGetLastError();
}

template <class T>
__global__ __launch_bounds__(256) void bfht_fill_zero(T* __restrict__ x, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) x[i] = from_f32<T>(0.0f);
}

__global__ __launch_bounds__(256) void bfht_sign_words_kernel(uint32_t seed32, int64_t block,
                                                              int layer, int64_t first_word,
                                                              int64_t nwords,
                                                              uint32_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < nwords)
    out[i] = sign_word(block_key(seed32, block), layer_key(layer), (uint32_t)(first_word + i));
}

// ---------------------------------------------------------------- tile passes

constexpr int kTileThreads = 1024;
constexpr int kTileElems = 1 << kTileLog;
constexpr int kTilePadded = kTileElems + (kTileElems >> 5);

// In-place unnormalized butterflies over tile-index bits [lo_bit, 15) of an
// LDS-resident 2^15 tile, in groups of up to 5 bits.
__device__ __forceinline__ void tile_fht_bits(float* lds, int tid, int lo_bit) {
  for (int lo = lo_bit; lo < kTileLog; lo += 5) {
    const int nb = kTileLog - lo < 5 ? kTileLog - lo : 5;
    float v[32];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 32; ++r) v[r] = lds[lds_index(group_pos<kTileLog, 5>(tid, r, lo, nb))];
    butterflies<32>(v, nb);
#pragma unroll
    for (int r = 0; r < 32; ++r) lds[lds_index(group_pos<kTileLog, 5>(tid, r, lo, nb))] = v[r];
  }
  __syncthreads();
}

// One tile pass.  `high` selects the pass kind; `src` and `dst` the fused
// prologue/epilogue (TileSrc / TileDst in bfht_launch.h).  Grid: one
// workgroup per (block slot, tile), 2^(LB-15) tiles per block.
template <class T>
__global__ __launch_bounds__(kTileThreads) void bfht_tile_pass(
    const T* __restrict__ src_io, float* __restrict__ work, T* __restrict__ dst_io, int LB,
    int high, int src, int dst, int n, int64_t first_block, int64_t start, int64_t stop,
    uint32_t seed32, int src_layer, int dst_layer) {
  __shared__ float lds[kTilePadded];
  const int tid = threadIdx.x;
  const int tiles_log = LB - kTileLog;
  const int64_t slot = (int64_t)blockIdx.x >> tiles_log;
  const int tile = (int)(blockIdx.x & ((1u << tiles_log) - 1));
  const int64_t block = first_block + slot;
  const int64_t B = (int64_t)1 << LB;
  const int64_t base = block * B;  // global coordinate of the block's position 0
  float* wblk = work + slot * B;
  const uint32_t bkey = block_key(seed32, block);
  const int col_log = kTileLog - tiles_log;  // high pass: columns per tile row

  // tile element e -> block position p
  auto pos = [&](int e) -> uint32_t {
    if (!high) return ((uint32_t)tile << kTileLog) | (uint32_t)e;
    const uint32_t row = (uint32_t)e >> col_log, col = (uint32_t)e & ((1u << col_log) - 1);
    return (row << kTileLog) | ((uint32_t)tile << col_log) | col;
  };

  const uint32_t skey = layer_key(src_layer);
#pragma unroll 4
  for (int r = 0; r < 32; ++r) {
    const int e = r * kTileThreads + tid;
    const uint32_t p = pos(e);
    float x;
    if (src == kSrcLatent) {
      x = (int)p < n ? to_f32(src_io[p]) : 0.0f;
    } else if (src == kSrcGrad) {
      const int64_t g = base + p;
      x = (g >= start && g < stop) ? to_f32(src_io[g - start]) : 0.0f;
    } else {
      x = wblk[p];
    }
    if (src != kSrcWork) x = signed_at(x, bkey, skey, p);
    lds[lds_index(e)] = x;
  }
  tile_fht_bits(lds, tid, high ? kTileLog - tiles_log : 0);

  const float scale = high ? ((LB & 1) ? 0.70710678118654752440f / (float)(1 << (LB >> 1))
                                       : 1.0f / (float)(1 << (LB >> 1)))
                           : 1.0f;
  const uint32_t dkey = layer_key(dst_layer);
#pragma unroll 4
  for (int r = 0; r < 32; ++r) {
    const int e = r * kTileThreads + tid;
    const uint32_t p = pos(e);
    float x = lds[lds_index(e)] * scale;
    if (dst == kDstWork) {
      wblk[p] = x;
    } else if (dst == kDstOut) {
      const int64_t g = base + p;
      if (g >= start && g < stop) dst_io[g - start] = from_f32<T>(signed_at(x, bkey, dkey, p));
    } else {  // kDstPartial: first n positions, signed by D_0, left in the work buffer
      if ((int)p < n) wblk[p] = signed_at(x, bkey, dkey, p);
    }
  }
}

// ---------------------------------------------------------------- launchers

template <int LB, class T>
static hipError_t launch_block_fwd(const BfhtArgs& a, hipStream_t s) {
  using Gm = Geo<LB>;
  const int64_t grid = (a.nblocks + Gm::G - 1) / Gm::G;
  hipLaunchKernelGGL((bfht_block_fwd<LB, T>), dim3((unsigned)grid), dim3(Gm::WG), 0, s,
                     (const T*)a.src, (T*)a.dst, (int)a.n, a.first_block, a.nblocks, a.start,
                     a.stop, a.seed32, a.layers);
  return hipGetLastError();
}

template <int LB, class T>
static hipError_t launch_block_bwd(const BfhtArgs& a, hipStream_t s) {
  using Gm = Geo<LB>;
  const int64_t grid = (a.nblocks + Gm::G - 1) / Gm::G;
  const int direct = a.nblocks == 1;
  hipLaunchKernelGGL((bfht_block_bwd<LB, T>), dim3((unsigned)grid), dim3(Gm::WG), 0, s,
                     (const T*)a.src, (float*)a.work, (T*)a.dst, (int)a.n, a.first_block,
                     a.nblocks, a.start, a.stop, a.seed32, a.layers, direct);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || direct) return e;
  return launch_reduce<T>((const float*)a.work, a.nblocks, a.n, a.n, (T*)a.dst, s);
}

template <class T>
using BlockLauncher = hipError_t (*)(const BfhtArgs&, hipStream_t);

template <class T, int... LBs>
static hipError_t dispatch_block(int LB, bool fwd, const BfhtArgs& a, hipStream_t s,
                                 std::integer_sequence<int, LBs...>) {
  static const BlockLauncher<T> fwd_table[] = {&launch_block_fwd<LBs, T>...};
  static const BlockLauncher<T> bwd_table[] = {&launch_block_bwd<LBs, T>...};
  return fwd ? fwd_table[LB](a, s) : bwd_table[LB](a, s);
}

template <class T>
static hipError_t run_tiles(const BfhtArgs& a, hipStream_t s, bool fwd) {
  const unsigned grid = (unsigned)(a.nblocks << (a.log_block - kTileLog));
  const int L = a.layers;
  for (int step = 0; step < L; ++step) {
    // forward layer l = step: D_l at the low pass' load, D_L at the last store.
    // backward layer l = L-1-step: D_{l+1} at the low pass' load, D_0 at the last store.
    const int layer = fwd ? step : L - 1 - step;
    const int low_src = step == 0 ? (fwd ? kSrcLatent : kSrcGrad) : kSrcWorkSigned;
    const int low_src_layer = fwd ? layer : layer + 1;
    hipLaunchKernelGGL((bfht_tile_pass<T>), dim3(grid), dim3(kTileThreads), 0, s,
                       (const T*)a.src, (float*)a.work, (T*)nullptr, a.log_block, 0, low_src,
                       kDstWork, (int)a.n, a.first_block, a.start, a.stop, a.seed32, low_src_layer,
                       0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const bool last = step == L - 1;
    const int hdst = last ? (fwd ? kDstOut : kDstPartial) : kDstWork;
    const int hdst_layer = fwd ? L : 0;
    hipLaunchKernelGGL((bfht_tile_pass<T>), dim3(grid), dim3(kTileThreads), 0, s,
                       (const T*)nullptr, (float*)a.work, (T*)a.dst, a.log_block, 1, kSrcWork, hdst,
                       (int)a.n, a.first_block, a.start, a.stop, a.seed32, 0, hdst_layer);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (fwd) return hipSuccess;
  return launch_reduce<T>((const float*)a.work, a.nblocks, (int64_t)1 << a.log_block, a.n, (T*)a.dst, s);
}

template <class T>
static hipError_t run_typed(const BfhtArgs& a, hipStream_t s, bool fwd) {
  if (a.nblocks == 0) {
    if (fwd) return hipSuccess;
    hipLaunchKernelGGL((bfht_fill_zero<T>), dim3((unsigned)((a.n + 255) / 256)), dim3(256), 0, s,
                       (T*)a.dst, a.n);
    return hipGetLastError();
  }
  if (mfma15_applicable(a)) {
    hipError_t e = launch_mfma15(a, s, fwd);
    if (e != hipSuccess || fwd) return e;
    return launch_reduce<T>((const float*)a.work, a.nblocks, a.n, a.n, (T*)a.dst, s);
  }
  if (a.log_block <= kTileLog)
    return dispatch_block<T>(a.log_block, fwd, a, s, std::make_integer_sequence<int, kTileLog + 1>{});
  return run_tiles<T>(a, s, fwd);
}

hipError_t launch_bfht(const BfhtArgs& a, hipStream_t s, bool forward) {
  switch (a.dtype) {
    case kF32: return run_typed<float>(a, s, forward);
    case kF16: return run_typed<f16>(a, s, forward);
    case kBF16: return run_typed<bf16>(a, s, forward);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_sign_words(uint32_t seed32, int64_t block, int layer, int64_t first_word,
                             int64_t nwords, uint32_t* out, hipStream_t s) {
  if (nwords <= 0) return hipSuccess;
  hipLaunchKernelGGL(bfht_sign_words_kernel, dim3((unsigned)((nwords + 255) / 256)), dim3(256), 0,
                     s, seed32, block, layer, first_word, nwords, out);
  return hipGetLastError();
}

}  // namespace lwl
