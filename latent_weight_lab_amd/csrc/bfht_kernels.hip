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
#include "bfht_block.h"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace lwl {

// Element access of the per-generator launches: the slice in the latent dtype.
// Element access of the per-generator launches: the slice in the latent dtype,
// through a buffer resource over one block's range (`range` + call) or by
// element index (`at`, for blocks that share a wave).
template <class T>
struct SliceStore {
  T* out;
  __device__ __amdgpu_buffer_rsrc_t range(int64_t first, int64_t count) const {
    return tile_rsrc(out + first, (uint64_t)count * sizeof(T));
  }
  __device__ void operator()(__amdgpu_buffer_rsrc_t r, int i, float v) const { buf_store<T>(v, r, i); }
  __device__ void whole(__amdgpu_buffer_rsrc_t r, int base, int c, float v) const { buf_store_at<T>(v, r, base, c); }
  __device__ void at(int64_t i, float v) const { out[i] = from_f32<T>(v); }
};
template <class T>
struct SliceLoad {
  const T* g;
  __device__ __amdgpu_buffer_rsrc_t range(int64_t first, int64_t count) const {
    return tile_rsrc(g + first, (uint64_t)count * sizeof(T));
  }
  __device__ float operator()(__amdgpu_buffer_rsrc_t r, int i) const { return buf_load<T>(r, i); }
  __device__ float whole(__amdgpu_buffer_rsrc_t r, int base, int c) const { return buf_load_at<T>(r, base, c); }
  __device__ float at(int64_t i) const { return to_f32(g[i]); }
};

template <int LB, class T>
__global__ __launch_bounds__(Geo<LB>::WG) void bfht_block_fwd(const T* __restrict__ latent, T* __restrict__ out,
                                                             int n, int64_t first_block, int64_t nblocks,
                                                             int64_t start, int64_t stop, uint32_t seed32,
                                                             int layers) {
  __shared__ float smem[BlockLds<LB>::FLOATS];
  const int64_t slot = (int64_t)blockIdx.x * Geo<LB>::G + (threadIdx.x >> Geo<LB>::LT);
  block_fwd_slot<LB, T>(latent, SliceStore<T>{out}, n, first_block, slot, nblocks, start, stop, seed32, layers,
                        smem);
}

template <int LB, class T>
__global__ __launch_bounds__(Geo<LB>::WG) void bfht_block_bwd(const T* __restrict__ grad,
                                                             float* __restrict__ partial,
                                                             T* __restrict__ grad_latent, int n,
                                                             int64_t first_block, int64_t nblocks, int64_t start,
                                                             int64_t stop, uint32_t seed32, int layers,
                                                             int direct) {
  __shared__ float smem[BlockLds<LB>::FLOATS];
  const int64_t slot = (int64_t)blockIdx.x * Geo<LB>::G + (threadIdx.x >> Geo<LB>::LT);
  block_bwd_slot<LB, T>(SliceLoad<T>{grad}, partial, n, grad_latent, n, first_block, slot, nblocks, start, stop,
                        seed32, layers, direct, smem);
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
constexpr int kRedDepth = 16;  // row loads in flight per wave (32 when a wave has more than 16 rows)

template <int kVec>
struct RedVec;
template <>
struct RedVec<1> { typedef float type; };
template <>
struct RedVec<2> { typedef float2 type; };
template <>
struct RedVec<4> { typedef float4 type; };

// Columns c0 .. c0 + kVec - 1 of the sum (kVec-wide loads when the row stride
// allows); every thread of the workgroup calls it, and wave 0 returns true with
// the totals.  Wave w adds rows w, w + 8, w + 16, ... in ascending order with
// kDepth row loads in flight (rows past the end are loaded from row 0 and
// not added, so the loads need no branch), and wave 0 adds the 8 wave sums in
// wave order: the result does not depend on kVec, kDepth or timing.
// kVec partial-row elements of type P, loaded together and widened to float
template <class P, int kVec>
struct PartVec;
template <int kVec>
struct PartVec<float, kVec> {
  typedef typename RedVec<kVec>::type type;
  static __device__ float at(const type& v, int e) {
    if constexpr (kVec == 1) return v;
    else return reinterpret_cast<const float*>(&v)[e];
  }
};
template <int kVec>
struct PartVec<bf16, kVec> {  // kVec bf16 = 2, 4 or 8 bytes
  typedef typename std::conditional<kVec == 1, uint16_t,
                                    typename std::conditional<kVec == 2, uint32_t, uint2>::type>::type type;
  static __device__ float at(const type& v, int e) {
    return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(&v)[e] << 16);
  }
};

// Load of data read exactly once (partial rows): nt cache policy, so the
// stream does not keep lines for reuse (config-2 bf16 backward 16.9 -> 15.4 us).
template <class V>
__device__ __forceinline__ V load_once(const V* p) {
  typedef uint32_t w2 __attribute__((ext_vector_type(2)));
  typedef uint32_t w4 __attribute__((ext_vector_type(4)));
  if constexpr (sizeof(V) == 2) return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p)));
  else if constexpr (sizeof(V) == 4) return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p)));
  else if constexpr (sizeof(V) == 8) return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const w2*>(p)));
  else return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const w4*>(p)));
}

template <int kVec, class P = float, int kDepth = kRedDepth>
__device__ __forceinline__ bool reduce_columns(const P* __restrict__ part, int64_t nblocks, int64_t stride,
                                               int n, int c0, float (&sums)[kRedWaves][kVec][64],
                                               float (&t)[kVec]) {
  typedef typename PartVec<P, kVec>::type V;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float a[kVec];
#pragma unroll
  for (int e = 0; e < kVec; ++e) a[e] = 0.0f;
  auto lanes = [](const V& v, int e) -> float { return PartVec<P, kVec>::at(v, e); };
  if (c0 + kVec <= n) {
    // every column of the lane is in range: vector loads
    for (int64_t b0 = wave; b0 < nblocks; b0 += (int64_t)kRedWaves * kDepth) {
      V v[kDepth];
#pragma unroll
      for (int j = 0; j < kDepth; ++j) {
        const int64_t b = b0 + (int64_t)kRedWaves * j;
        v[j] = load_once(reinterpret_cast<const V*>(part + (b < nblocks ? b : 0) * stride + c0));
      }
      // every load issued before the first add: left to itself the compiler
      // issues them in batches of eight and waits out each batch
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < kDepth; ++j) {
        const bool ok = b0 + (int64_t)kRedWaves * j < nblocks;
#pragma unroll
        for (int e = 0; e < kVec; ++e) a[e] = ok ? a[e] + lanes(v[j], e) : a[e];
      }
    }
  } else {
    // the tail of the row: element loads, columns past n read column 0
    for (int64_t b0 = wave; b0 < nblocks; b0 += (int64_t)kRedWaves * kRedDepth) {
      float v[kRedDepth][kVec];
#pragma unroll
      for (int j = 0; j < kRedDepth; ++j) {
        const int64_t b = b0 + (int64_t)kRedWaves * j;
        const P* r = part + (b < nblocks ? b : 0) * stride;
#pragma unroll
        for (int e = 0; e < kVec; ++e) v[j][e] = to_f32(r[c0 + e < n ? c0 + e : 0]);
      }
#pragma unroll
      for (int j = 0; j < kRedDepth; ++j) {
        const bool ok = b0 + (int64_t)kRedWaves * j < nblocks;
#pragma unroll
        for (int e = 0; e < kVec; ++e) a[e] = ok ? a[e] + v[j][e] : a[e];
      }
    }
  }
#pragma unroll
  for (int e = 0; e < kVec; ++e) sums[wave][e][lane] = a[e];
  __syncthreads();
  if (wave != 0) return false;
#pragma unroll
  for (int e = 0; e < kVec; ++e) {
    t[e] = 0.0f;
#pragma unroll
    for (int w = 0; w < kRedWaves; ++w) t[e] += sums[w][e][lane];
  }
  return true;
}

template <class T, int kVec, class P = float, int kDepth = kRedDepth>
__global__ __launch_bounds__(64 * kRedWaves) void bfht_reduce_blocks(const P* __restrict__ part,
                                                                     int64_t nblocks, int64_t stride, int n,
                                                                     T* __restrict__ grad_latent) {
  __shared__ float sums[kRedWaves][kVec][64];
  const int c0 = (blockIdx.x * 64 + (threadIdx.x & 63)) * kVec;
  float t[kVec];
  if (!reduce_columns<kVec, P, kDepth>(part, nblocks, stride, n, c0, sums, t)) return;
#pragma unroll
  for (int e = 0; e < kVec; ++e)
    if (c0 + e < n) grad_latent[c0 + e] = from_f32<T>(t[e]);
}

// Few rows (nblocks <= kRedWaves): one thread per kVec columns adds the rows
// in ascending order with all of its loads in flight.  That is the wave-split
// kernel's sum exactly (there wave w holds row w alone, and the wave sums are
// added in wave order onto 0), without its one load in flight per lane.
// Rows past nblocks are loaded from row 0 and not added; with no rows at all
// (part may then be null) nothing is loaded and the sum is 0.
template <class T, int kVec, class P>
__global__ __launch_bounds__(256) void bfht_reduce_few(const P* __restrict__ part, int nblocks, int64_t stride,
                                                       int n, T* __restrict__ grad_latent) {
  typedef typename PartVec<P, kVec>::type V;
  const int c0 = (blockIdx.x * 256 + (int)threadIdx.x) * kVec;
  if (c0 >= n) return;
  float a[kVec];
#pragma unroll
  for (int e = 0; e < kVec; ++e) a[e] = 0.0f;
  if (nblocks <= 0) {
    // no partial rows: a zero gradient
  } else if (c0 + kVec <= n) {
    V v[kRedWaves];
#pragma unroll
    for (int b = 0; b < kRedWaves; ++b) v[b] = load_once(reinterpret_cast<const V*>(part + (b < nblocks ? b : 0) * stride + c0));
#pragma unroll
    for (int b = 0; b < kRedWaves; ++b)
#pragma unroll
      for (int e = 0; e < kVec; ++e) a[e] = b < nblocks ? a[e] + PartVec<P, kVec>::at(v[b], e) : a[e];
  } else {
#pragma unroll
    for (int b = 0; b < kRedWaves; ++b) {
      const P* r = part + (b < nblocks ? b : 0) * stride;
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        const float v = to_f32(r[c0 + e < n ? c0 + e : 0]);
        a[e] = b < nblocks ? a[e] + v : a[e];
      }
    }
  }
#pragma unroll
  for (int e = 0; e < kVec; ++e)
    if (c0 + e < n) grad_latent[c0 + e] = from_f32<T>(a[e]);
}

// Grouped block sums with the flush epilogue: r = T(T(sum) * scale), added to
// the destination in T when the job accumulates.  Rows are 128-byte aligned
// (the planner rounds the stride up to 32 floats), so loads are 16 bytes wide.
template <class T>
__device__ __forceinline__ void grad_store(T* dst, int i, float sum, float scale, int accumulate, float prev) {
  float r = round_to<T>(round_to<T>(sum) * scale);
  if (accumulate) r = prev + r;  // prev: dst[i] as float
  dst[i] = from_f32<T>(r);
}

template <class T, class P>
__global__ __launch_bounds__(64 * kRedWaves) void bfht_reduce_grouped(const GroupTable g) {
  static_assert(kGroupReduceCols == 64 * 4, "grouped prefix counts reduce tiles of 4 columns per lane");
  __shared__ float sums[kRedWaves][4][64];
  const int j = group_job(g, (int)blockIdx.x);
  const GroupJob& jb = g.job[j];
  const int n = jb.n;
  const int c0 = ((blockIdx.x - g.prefix[j]) * 64 + (threadIdx.x & 63)) * 4;
  float t[4];
  if (!reduce_columns<4, P>(static_cast<const P*>(jb.part), jb.nblocks, jb.stride, n, c0, sums, t)) return;
  T* dst = static_cast<T*>(jb.dst);
  // an accumulating job reads its four destination values together first
  // (each read behind its own column check was waited out on its own)
  float prev[4] = {0.f, 0.f, 0.f, 0.f};
  if (jb.accumulate) {
#pragma unroll
    for (int e = 0; e < 4; ++e) prev[e] = c0 + e < n ? to_f32(dst[c0 + e]) : 0.f;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (c0 + e < n) grad_store<T>(dst, c0 + e, t[e], jb.scale, jb.accumulate, prev[e]);
}

template <class T, int kVec, class P>
static void launch_reduce_vec(const P* part, int64_t nblocks, int64_t stride, int64_t n, T* dst, hipStream_t s) {
  if (nblocks <= kRedWaves) {
    const dim3 grid((unsigned)((n + 256 * kVec - 1) / (256 * kVec))), block(256);
    hipLaunchKernelGGL((bfht_reduce_few<T, kVec, P>), grid, block, 0, s, part, (int)nblocks, stride, (int)n, dst);
    return;
  }
  const dim3 grid((unsigned)((n + 64 * kVec - 1) / (64 * kVec))), block(64 * kRedWaves);
  // More than 16 rows per wave (config 2: 256 rows, 32 per wave): all of a
  // wave's row loads in one round instead of two memory round trips.
  if (nblocks > (int64_t)kRedWaves * kRedDepth)
    hipLaunchKernelGGL((bfht_reduce_blocks<T, kVec, P, 2 * kRedDepth>), grid, block, 0, s, part, nblocks, stride,
                       (int)n, dst);
  else
    hipLaunchKernelGGL((bfht_reduce_blocks<T, kVec, P>), grid, block, 0, s, part, nblocks, stride, (int)n, dst);
}

template <class T, class P = float>
static hipError_t launch_reduce(const P* part, int64_t nblocks, int64_t stride, int64_t n, T* dst,
                                hipStream_t s) {
  // The widest row loads the stride allows (part is 256-byte aligned) that still
  // give every CU a workgroup: 64 * kVec columns per workgroup (256 * kVec with
  // few rows, where a thread takes every row of its columns).
  const int64_t per = nblocks <= kRedWaves ? 256 : 64;
  auto fits = [&](int v) { return stride % v == 0 && (n + per * v - 1) / (per * v) >= 256; };
  if (fits(4))
    launch_reduce_vec<T, 4>(part, nblocks, stride, n, dst, s);
  else if (fits(2))
    launch_reduce_vec<T, 2>(part, nblocks, stride, n, dst, s);
  else
    launch_reduce_vec<T, 1>(part, nblocks, stride, n, dst, s);
  return hipGetLastError();
}

hipError_t launch_block_sum(const float* part, int64_t rows, int64_t stride, int64_t n, void* dst, int dtype,
                            hipStream_t s) {
  switch (dtype) {
    case kF32: return launch_reduce<float>(part, rows, stride, n, (float*)dst, s);
    case kF16: return launch_reduce<f16>(part, rows, stride, n, (f16*)dst, s);
    case kBF16: return launch_reduce<bf16>(part, rows, stride, n, (bf16*)dst, s);
  }
  return hipErrorInvalidValue;
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

// Bit groups of a tile pass that transforms tile-index bits [LO_BIT, 15): the
// register bits of the load layout (element r * 1024 + tid holds bits 10-14
// in r; those at or above LO_BIT, from register bit kRegLo), then [LO_BIT, 10)
// in at most two groups of up to 5 bits from the top.
template <int LO_BIT>
struct TileGroups {
  static constexpr int kRegLo = LO_BIT > 10 ? LO_BIT - 10 : 0;
  static constexpr int kExtra = LO_BIT >= 10 ? 0 : (10 - LO_BIT + 4) / 5;
  static constexpr int lo(int k) { return 10 - 5 * k - 5 > LO_BIT ? 10 - 5 * k - 5 : LO_BIT; }
  static constexpr int nb(int k) { return 10 - 5 * k - lo(k); }
  // the layout after the groups: the last extra group, or the load layout (10, 5)
  static constexpr int kLastLo = kExtra == 0 ? 10 : lo(kExtra - 1);
  static constexpr int kLastNb = kExtra == 0 ? 5 : nb(kExtra - 1);
};
static_assert(TileGroups<0>::kExtra == 2 && TileGroups<0>::lo(0) == 5 && TileGroups<0>::lo(1) == 0 &&
                  TileGroups<0>::nb(1) == 5,
              "low tile: bits 10-14 in registers, then 5-9 and 0-4");
static_assert(TileGroups<7>::kExtra == 1 && TileGroups<7>::lo(0) == 7 && TileGroups<7>::nb(0) == 3,
              "2^23 high tile: bits 10-14 in registers, then 7-9");
static_assert(TileGroups<10>::kExtra == 0 && TileGroups<12>::kRegLo == 2, "small high tiles stay in registers");


// Sign layer in bit-group layout (L, NB): element e = group_pos(tid, r, L, NB)
// takes bit e & 31 of table word e >> 5.
// In chunks of 8 registers, each chunk's table reads kept behind the previous
// chunk's flips (at most 8 words in registers beside the tile and the loads
// in flight for the next one).
template <int L, int NB>
__device__ __forceinline__ void tile_signs(const uint32_t* words, float (&v)[32], int tid) {
#pragma unroll
  for (int r0 = 0; r0 < 32; r0 += 8) {
#pragma unroll
    for (int r = r0; r < r0 + 8; ++r) {
      const int e = group_pos<kTileLog, 5>(tid, r, L, NB);
      v[r] = signed_by(v[r], words[e >> 5], e & 31);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The same for a group below bit 10 (L >= 5): the thread's and the register's
// bit fields of e are disjoint and the register's lie at bit 5 and above, so
// every register takes the same bit of the words at the thread's base plus a
// constant per register (immediate LDS offsets, no per-register index work).
template <int L, int NB>
__device__ __forceinline__ void tile_signs_split(const uint32_t* words, float (&v)[32], int tid) {
  static_assert(L >= 5, "the bit within a sign word comes from the thread index alone");
  const int e0 = group_pos<kTileLog, 5>(tid, 0, L, NB);
  const uint32_t* w = words + (e0 >> 5);
  const int bit = e0 & 31;
#pragma unroll
  for (int r0 = 0; r0 < 32; r0 += 8) {
#pragma unroll
    for (int r = r0; r < r0 + 8; ++r) v[r] = signed_by(v[r], w[group_pos<kTileLog, 5>(0, r, L, NB) >> 5], bit);
    __builtin_amdgcn_sched_barrier(0);
  }
}
// group_pos(t, r, L, NB) = group_pos(t, 0, L, NB) | group_pos(0, r, L, NB) for L >= 5, as tile_signs_split uses it
constexpr bool tile_signs_split_ok() {
  for (int L = 5; L <= 10; ++L)
    for (int NB = 1; NB <= 5 && L + NB <= 15; ++NB)
      for (int i = 0; i < 14; ++i)
        for (int r = 0; r < 32; ++r) {
          // every single thread-index bit, none, all, and two mixed patterns
          const int t = i < 10 ? 1 << i : i == 10 ? 0 : i == 11 ? kTileThreads - 1 : i == 12 ? 0x155 : 0x2aa;
          const int e = group_pos<kTileLog, 5>(t, r, L, NB), a = group_pos<kTileLog, 5>(t, 0, L, NB),
                    b = group_pos<kTileLog, 5>(0, r, L, NB);
          if (e != (a | b) || (a & b) != 0 || (b & 31) != 0) return false;
        }
  return true;
}
static_assert(tile_signs_split_ok(), "tile_signs_split's split of the element index");

// Butterflies over register bits [LO, 5).
template <int LO>
__device__ __forceinline__ void reg_butterflies(float (&v)[32]) {
#pragma unroll
  for (int j = LO; j < 5; ++j)
#pragma unroll
    for (int r = 0; r < 32; ++r)
      if (!(r & (1 << j))) {
        const float a = v[r], b = v[r | (1 << j)];
        v[r] = a + b;
        v[r | (1 << j)] = a - b;
      }
}


// One pass of the tiled schedule (run_tiles).  A tile is 2^15 positions of one
// block (in registers, through LDS between bit groups): a low tile is
// contiguous (block bits 0-14 vary), a high
// tile is 2^(LB-15) rows of 2^(30-LB) contiguous columns, the rows walking
// block bits 15..LB-1.  The pass loads the tile (latent, grad or the work
// buffer), transforms its bit group (`pre`), applies the sign layer
// `sign_layer`, transforms the same bit group again (`post`), scales, and
// stores it (work buffer, output slice, or partial gradient row).  Each thread
// hashes one of the tile's 1024 sign words into a shared table.  Tiles are
// numbered slot * 2^(LB-15) + tile (2^(LB-15) tiles per block slot); the grid is
// persistent (one workgroup per CU walks tiles blockIdx.x, + gridDim.x, ...) and
// loads the next tile into registers while it transforms the current one, so a
// CU's loads, transforms and stores overlap.
//
// Element r * 1024 + tid of the tile sits at block position pt(tid) + pr(r)
// (disjoint bit fields), so each thread keeps one 32-bit offset and adds a
// wave-uniform one per register: the 32 loads are issued back to back without
// per-element addresses, and range limits (latent length, slice ends) are
// buffer bounds.  SRC / DST are compile-time.
//
// DST = kDstSum (the backward's last pass): instead of one partial row per
// block, workgroup (tile, group) walks tile `tile` of the group's blocks
// group * group_blocks .. in ascending order (the next block's tile loading
// while the current one transforms) and adds each block's scaled result in
// registers; at the end it stores the sum of its group: straight to the latent
// gradient (dst_io, the first n positions) when there is one group, else into
// the work buffer's row of the group's first block (read by no other
// workgroup, and by this one before it is written), for the block sum over
// the groups.
template <class T, int SRC, int DST, int TL>
__global__ __launch_bounds__(kTileThreads) void bfht_tile_pass(
    const T* __restrict__ src_io, float* __restrict__ work, T* __restrict__ dst_io, int LB, int pre, int post,
    int n, int64_t first_block, int64_t ntiles_total, int64_t start, int64_t stop, uint32_t seed32, int sign_layer,
    float scale, int64_t group_blocks, int ngroups) {
  __shared__ float lds[kTilePadded];
  __shared__ uint32_t words[kTileElems / 32];
  static_assert(kTileElems / 32 == kTileThreads, "one sign word per thread");
  // TL = 0: low tile; TL = LB - 15 (the launcher checks): high tile of 2^TL rows
  constexpr bool high = TL > 0;
  const int tid = threadIdx.x;
  const int tiles_log = LB - kTileLog;  // log2 tiles per block
  const int64_t B = (int64_t)1 << LB;
  constexpr int col_log = kTileLog - TL;  // high tile: columns per row (>= 7 for LB <= 23)
  constexpr int lo_bit = high ? col_log : 0;  // the tile-index bits the pass transforms

  // tile element e -> block position; elements 32q .. 32q+31 are positions
  // pos(32q) .. pos(32q)+31 (columns are at least 32 wide)
  auto pos = [&](uint32_t e, int tile) -> uint32_t {
    if (!high) return ((uint32_t)tile << kTileLog) | e;
    const uint32_t row = e >> col_log, col = e & ((1u << col_log) - 1);
    return (row << kTileLog) | ((uint32_t)tile << col_log) | col;
  };
  // pos(r * 1024 + tid) = pos(tid) + pr(r): the register's field does not depend on the tile
  auto pr = [&](int r) { return (int)pos((uint32_t)r * kTileThreads, 0); };

  struct Geo {
    int64_t slot, block, base, lo, hi;  // block-local slice range [lo, hi) (grad / out)
    int tile, pt;
  };
  auto geo = [&](int64_t t) {
    Geo g;
    g.slot = t >> tiles_log;
    g.tile = (int)(t & ((1 << tiles_log) - 1));
    g.block = first_block + g.slot;
    g.base = g.block * B;
    g.lo = start - g.base > 0 ? start - g.base : 0;
    g.hi = stop - g.base < B ? stop - g.base : B;
    g.pt = (int)pos((uint32_t)tid, g.tile);
    return g;
  };
  // A tile wholly inside its buffer (the work buffer always; the latent when
  // it covers the block, a gradient or output slice when it covers the whole
  // block) is accessed at the thread's offset plus each register's constant
  // one in the scalar offset, with no per-element range arithmetic (about a
  // fifth of a low tile's VALU work otherwise); other tiles check every index.
  auto load_tile = [&](const Geo& g, float (&x)[32]) {
    if constexpr (SRC == kSrcLatent) {
      const auto lr = tile_rsrc(src_io, (uint64_t)n * sizeof(T));
      if (n >= B) {
#pragma unroll
        for (int r = 0; r < 32; ++r) x[r] = buf_load_at<T>(lr, g.pt, pr(r));
      } else {
#pragma unroll
        for (int r = 0; r < 32; ++r) x[r] = buf_load<T>(lr, g.pt + pr(r));
      }
    } else if constexpr (SRC == kSrcGrad) {
      // buffer over grad[lo..hi) of this block, indexed by block position - lo
      const T* g0 = src_io + (g.base + g.lo - start);
      const auto gr = tile_rsrc(g0, (uint64_t)(g.hi - g.lo) * sizeof(T));
      if (g.lo == 0 && g.hi == B) {
#pragma unroll
        for (int r = 0; r < 32; ++r) x[r] = buf_load_at<T>(gr, g.pt, pr(r));
      } else {
#pragma unroll
        for (int r = 0; r < 32; ++r) x[r] = buf_load<T>(gr, g.pt + pr(r) - (int)g.lo);
      }
    } else {
      const auto wr = tile_rsrc(work + g.slot * B, (uint64_t)B * 4);
#pragma unroll
      for (int r = 0; r < 32; ++r) x[r] = buf_load_at<float>(wr, g.pt, pr(r));
    }
  };

  // Bit groups (TileGroups): the load layout's register bits (element
  // r * 1024 + tid), then the groups below bit 10 through LDS.  A tile with no
  // group below bit 10 stays in registers from load to store.  Otherwise the
  // first transform starts on the loaded registers, the tile goes to LDS once
  // (freeing the registers for the next tile's loads) and visits the groups
  // downwards; the sign layer is applied in the last group's layout — for a low
  // tile 32 consecutive positions, one sign word, the thread's own — and the
  // second transform visits the groups upwards and ends in the load layout,
  // stored from registers.  Per group: a barrier, a read, the butterflies, a
  // write back of the same elements.
  using G = TileGroups<lo_bit>;
  constexpr bool kOwnWord = G::kLastLo == 0 && G::kLastNb == 5;  // 32 consecutive positions per thread
  auto group_rw = [&](float (&v)[32], int lo, int nb, bool rd) {
    const int b = group_base<kTileLog, 5>(tid, lo, nb);
    if (rd) {
#pragma unroll
      for (int r = 0; r < 32; ++r) v[r] = lds[group_lds<kTileLog, 5>(b, r, lo, nb)];
    } else {
#pragma unroll
      for (int r = 0; r < 32; ++r) lds[group_lds<kTileLog, 5>(b, r, lo, nb)] = v[r];
    }
  };
  // the tiles this workgroup walks: t0, t0 + t_step, ... below t_end
  int64_t t0 = blockIdx.x, t_step = gridDim.x, t_end = ntiles_total;
  int sum_tile = 0;
  int64_t sum_group = 0;
  float acc[32];
  if constexpr (DST == kDstSum) {
    sum_tile = (int)(blockIdx.x & ((1u << tiles_log) - 1));
    sum_group = (int64_t)(blockIdx.x >> tiles_log);
    const int64_t nblk = ntiles_total >> tiles_log;
    const int64_t b0 = sum_group * group_blocks;
    const int64_t b1 = b0 + group_blocks < nblk ? b0 + group_blocks : nblk;
    t0 = (b0 << tiles_log) | sum_tile;
    t_step = (int64_t)1 << tiles_log;
    t_end = b1 << tiles_log;
#pragma unroll
    for (int r = 0; r < 32; ++r) acc[r] = 0.0f;
  }
  // The next tile's loads are in flight during the current one's transforms,
  // except in a summing pass over high tiles that go through LDS (blocks above
  // 2^20): there the sum's 32 registers leave no room for them beside the
  // transform's, and each tile is loaded at the start of its own iteration.
  constexpr bool kPrefetch = !(DST == kDstSum && high && G::kExtra > 0);
  float x[32];
  int64_t t = t0;
  if (kPrefetch && t < t_end) load_tile(geo(t), x);
  for (; t < t_end; t += t_step) {
    const Geo g = geo(t);
    if constexpr (!kPrefetch) load_tile(g, x);
    float v[32];
    __syncthreads();  // the previous tile's reads of lds and of the sign table are done
    const uint32_t my_word = sign_word(block_key(seed32, g.block), layer_key(sign_layer), pos(32u * tid, g.tile) >> 5);
    words[tid] = my_word;
    if constexpr (G::kExtra == 0) {
#pragma unroll
      for (int r = 0; r < 32; ++r) v[r] = x[r];
      if (t + t_step < t_end) load_tile(geo(t + t_step), x);  // in flight during the transforms
      if (pre) reg_butterflies<G::kRegLo>(v);
      __syncthreads();  // the sign table is complete
      tile_signs<10, 5>(words, v, tid);
      if (post) reg_butterflies<G::kRegLo>(v);
    } else {
      if (pre) reg_butterflies<G::kRegLo>(x);
      group_rw(x, 10, 5, false);
      if (kPrefetch && t + t_step < t_end) load_tile(geo(t + t_step), x);  // in flight during the transforms
      // downwards: the groups of the first transform (without one, straight to
      // the last group's layout), then the sign layer
      if (pre) {
#pragma unroll
        for (int k = 0; k < G::kExtra; ++k) {
          __syncthreads();
          group_rw(v, G::lo(k), G::nb(k), true);
          butterflies<32>(v, G::nb(k));
          if (k + 1 < G::kExtra) group_rw(v, G::lo(k), G::nb(k), false);
        }
      } else {
        __syncthreads();
        group_rw(v, G::kLastLo, G::kLastNb, true);
      }
      if constexpr (kOwnWord) {
#pragma unroll
        for (int r = 0; r < 32; ++r) v[r] = signed_by(v[r], my_word, r);
      } else {
        // a high tile's small group below bit 10.  A middle pass (work buffer to
        // work buffer, transformed again after the signs) puts the signs on in
        // the group's layout (each element's word looked up by its tile index;
        // the table is complete: barriers since its writes).  The other passes
        // keep their register budget: the signs go on in the load layout (as in
        // a register-only tile), then back to the group if transformed again.
        bool in_group = false;
        if constexpr (DST == kDstWork) in_group = post != 0;
        if (in_group) {
          tile_signs_split<G::kLastLo, G::kLastNb>(words, v, tid);
        } else {
          group_rw(v, G::kLastLo, G::kLastNb, false);
          __syncthreads();
          group_rw(v, 10, 5, true);
          tile_signs<10, 5>(words, v, tid);
          if (post) {
            group_rw(v, 10, 5, false);
            __syncthreads();
            group_rw(v, G::kLastLo, G::kLastNb, true);
          }
        }
      }
      // upwards: the groups of the second transform (or only the way back); a
      // small high group without a second transform is in the load layout already
      if (kOwnWord || post) {
#pragma unroll
        for (int k = G::kExtra - 1; k >= 0; --k) {
          if (k + 1 < G::kExtra) {
            __syncthreads();
            group_rw(v, G::lo(k), G::nb(k), true);
          }
          if (post) butterflies<32>(v, G::nb(k));
          group_rw(v, G::lo(k), G::nb(k), false);
        }
        __syncthreads();
        group_rw(v, 10, 5, true);
        if (post) reg_butterflies<G::kRegLo>(v);
      }
    }

    if constexpr (DST == kDstSum) {
#pragma unroll
      for (int r = 0; r < 32; ++r) acc[r] += v[r] * scale;
    } else if constexpr (DST == kDstWork) {
      const auto wr = tile_rsrc(work + g.slot * B, (uint64_t)B * 4);
#pragma unroll
      for (int r = 0; r < 32; ++r) buf_store_at<float>(v[r] * scale, wr, g.pt, pr(r));
    } else {
      static_assert(DST == kDstOut, "tile pass destinations: work buffer, output slice, block sum");
      T* o0 = dst_io + (g.base + g.lo - start);
      const auto orr = tile_rsrc(o0, (uint64_t)(g.hi - g.lo) * sizeof(T));
      if (g.lo == 0 && g.hi == B) {
#pragma unroll
        for (int r = 0; r < 32; ++r) buf_store_at<T>(v[r] * scale, orr, g.pt, pr(r));
      } else {
#pragma unroll
        for (int r = 0; r < 32; ++r) buf_store<T>(v[r] * scale, orr, g.pt + pr(r) - (int)g.lo);
      }
    }
  }
  if constexpr (DST == kDstSum) {
    const int pt = (int)pos((uint32_t)tid, sum_tile);
    if (ngroups == 1) {
#pragma unroll
      for (int r = 0; r < 32; ++r) buf_store<T>(acc[r], tile_rsrc(dst_io, (uint64_t)n * sizeof(T)), pt + pr(r));
    } else {
      float* row = work + sum_group * group_blocks * B;
#pragma unroll
      for (int r = 0; r < 32; ++r) buf_store<float>(acc[r], tile_rsrc(row, (uint64_t)n * 4), pt + pr(r));
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

// One tile pass: picks the instantiation for (source, destination, tile kind).
// Passes that neither read nor write the I/O type run the float instantiation.
template <class T, int SRC, int DST>
static hipError_t launch_tile_kind(const BfhtArgs& a, hipStream_t s, int tl, int pre, int post, int layer,
                                   float scale, unsigned grid, int64_t group_blocks = 0, int ngroups = 0) {
  const int64_t ntiles = a.nblocks << (a.log_block - kTileLog);
  constexpr bool typed = SRC != kSrcWork || DST == kDstOut || DST == kDstSum;
  using U = std::conditional_t<typed, T, float>;
#define LWL_TILE(TL)                                                                                      \
  hipLaunchKernelGGL((bfht_tile_pass<U, SRC, DST, TL>), dim3(grid), dim3(kTileThreads), 0, s,            \
                     (const U*)a.src, (float*)a.work, (U*)a.dst, a.log_block, pre, post, (int)a.n,         \
                     a.first_block, ntiles, a.start, a.stop, a.seed32, layer, scale, group_blocks, ngroups)
  switch (tl) {
    case 0: LWL_TILE(0); break;
    case 1: if constexpr (SRC == kSrcWork) LWL_TILE(1); break;
    case 2: if constexpr (SRC == kSrcWork) LWL_TILE(2); break;
    case 3: if constexpr (SRC == kSrcWork) LWL_TILE(3); break;
    case 4: if constexpr (SRC == kSrcWork) LWL_TILE(4); break;
    case 5: if constexpr (SRC == kSrcWork) LWL_TILE(5); break;
    case 6: if constexpr (SRC == kSrcWork) LWL_TILE(6); break;
    case 7: if constexpr (SRC == kSrcWork) LWL_TILE(7); break;
    case 8: if constexpr (SRC == kSrcWork) LWL_TILE(8); break;
    default: return hipErrorInvalidValue;
  }
#undef LWL_TILE
  return hipGetLastError();
}

template <class T>
static hipError_t launch_tile_pass(const BfhtArgs& a, hipStream_t s, int src, int dst, int tl, int pre, int post,
                                   int layer, float scale, unsigned grid) {
  // the first pass (the only one reading latent / grad) runs low tiles
  if (src == kSrcLatent) return launch_tile_kind<T, kSrcLatent, kDstWork>(a, s, 0, pre, post, layer, scale, grid);
  if (src == kSrcGrad) return launch_tile_kind<T, kSrcGrad, kDstWork>(a, s, 0, pre, post, layer, scale, grid);
  if (dst == kDstWork) return launch_tile_kind<T, kSrcWork, kDstWork>(a, s, tl, pre, post, layer, scale, grid);
  return launch_tile_kind<T, kSrcWork, kDstOut>(a, s, tl, pre, post, layer, scale, grid);
}

// Blocks above 2^15: H = H_low (x) H_high over block bits 0-14 and 15..LB-1,
// the two factors commute, so consecutive layers share a pass:
//   [D_0, H_low] [H_high, D_1, H_high] [H_low, D_2, H_low] ... [H_g, D_L, out]
// (L + 1 passes, each one read and one write of the float32 work buffer).
// Pass k >= 1 completes layer k - 1 and applies its 2^(-LB/2).  The backward
// runs the same schedule on grad with the sign layers in reverse (D_L first,
// D_0 last); its last pass (kDstSum) also sums the blocks: each workgroup adds
// one tile position range over a group of blocks, with enough groups to give
// every CU a workgroup, and only with more than one group does a block sum
// over the groups' rows follow (config 3: 2^20 blocks, 64 blocks in 8 groups,
// 32 MiB of rows instead of 256 MiB; 2^23, 8 blocks in one group, no rows).
// Workgroups of the persistent tile passes: one per CU (a workgroup takes all
// of a CU's LDS), never more than the tiles.
// The CU count of the current device, cached per device: each slot is written
// with the same value by whichever thread gets there first (relaxed atomics,
// so concurrent callers need no lock).
constexpr int kMaxDevices = 64;
static std::atomic<int> g_cu_count[kMaxDevices];

static unsigned tile_grid(int64_t ntiles) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  if (dev >= 0 && dev < kMaxDevices) cus = g_cu_count[dev].load(std::memory_order_relaxed);
  if (cus <= 0) {
    int v = 0;
    cus = (dev >= 0 && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
              ? v
              : 256;
    if (dev >= 0 && dev < kMaxDevices) g_cu_count[dev].store(cus, std::memory_order_relaxed);
  }
  return (unsigned)std::min<int64_t>(ntiles, cus);
}

template <class T>
static hipError_t run_tiles(const BfhtArgs& a, hipStream_t s, bool fwd);

// Forward: the passes over one group of blocks after another (tile_group_blocks),
// each group a slice of the call's range, in the same work buffer.
template <class T>
static hipError_t run_tiles_grouped(const BfhtArgs& a, hipStream_t s) {
  const int64_t per = tile_group_blocks(a.log_block);
  if (a.nblocks <= per) return run_tiles<T>(a, s, true);
  const int64_t B = (int64_t)1 << a.log_block;
  for (int64_t b0 = 0; b0 < a.nblocks; b0 += per) {
    BfhtArgs g = a;
    g.first_block = a.first_block + b0;
    g.nblocks = std::min<int64_t>(per, a.nblocks - b0);
    g.start = std::max<int64_t>(a.start, g.first_block * B);
    g.stop = std::min<int64_t>(a.stop, (g.first_block + g.nblocks) * B);
    g.dst = static_cast<T*>(a.dst) + (g.start - a.start);
    const hipError_t e = run_tiles<T>(g, s, true);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <class T>
static hipError_t run_tiles(const BfhtArgs& a, hipStream_t s, bool fwd) {
  const int64_t tiles_per_block = (int64_t)1 << (a.log_block - kTileLog);
  const unsigned grid = tile_grid(a.nblocks * tiles_per_block);
  const int L = a.layers;
  const int LB = a.log_block;
  const float norm = (LB & 1) ? 0.70710678118654752440f / (float)(1 << (LB >> 1)) : 1.0f / (float)(1 << (LB >> 1));
  // the backward's summing last pass: groups of group_blocks blocks, one
  // workgroup per (tile, group), at least as many workgroups as CUs where the
  // blocks allow, no empty group
  const int64_t cus = tile_grid(INT64_MAX);
  int64_t ngroups = std::min<int64_t>(std::max<int64_t>((cus + tiles_per_block - 1) / tiles_per_block, 1), a.nblocks);
  const int64_t group_blocks = (a.nblocks + ngroups - 1) / ngroups;
  ngroups = (a.nblocks + group_blocks - 1) / group_blocks;
  for (int k = 0; k <= L; ++k) {
    const int src = k == 0 ? (fwd ? kSrcLatent : kSrcGrad) : kSrcWork;
    const int tl = (k & 1) ? LB - kTileLog : 0;  // odd passes run high tiles
    const float scale = k > 0 ? norm : 1.0f;
    hipError_t e;
    if (k == L && !fwd)
      e = launch_tile_kind<T, kSrcWork, kDstSum>(a, s, tl, (int)(k > 0), 0, 0, scale,
                                                  (unsigned)(tiles_per_block * ngroups), group_blocks, (int)ngroups);
    else
      e = launch_tile_pass<T>(a, s, src, k == L ? kDstOut : kDstWork, tl, (int)(k > 0), (int)(k < L),
                              fwd ? k : L - k, scale, grid);
    if (e != hipSuccess) return e;
  }
  if (fwd || ngroups == 1) return hipSuccess;
  return launch_reduce<T>((const float*)a.work, ngroups, group_blocks << a.log_block, a.n, (T*)a.dst, s);
}

template <class T>
static hipError_t run_typed(const BfhtArgs& a, hipStream_t s, bool fwd) {
  if (a.nblocks == 0) {
    if (fwd) return hipSuccess;
    hipLaunchKernelGGL((bfht_fill_zero<T>), dim3((unsigned)((a.n + 255) / 256)), dim3(256), 0, s,
                       (T*)a.dst, a.n);
    return hipGetLastError();
  }
  if (mfma15_applicable(a, fwd)) {
    hipError_t e = launch_mfma15(a, s, fwd);
    if (e != hipSuccess || fwd) return e;
    return launch_reduce<T, bf16>((const bf16*)a.work, a.nblocks, mfma15_part_stride(a.n), a.n, (T*)a.dst, s);
  }
  if (a.log_block <= kTileLog)
    return dispatch_block<T>(a.log_block, fwd, a, s, std::make_integer_sequence<int, kTileLog + 1>{});
  return fwd ? run_tiles_grouped<T>(a, s) : run_tiles<T>(a, s, false);
}

hipError_t launch_reduce_grouped(const GroupTable& g, int dtype, bool part_bf16, hipStream_t s) {
  if (g.count <= 0 || g.prefix[g.count] == 0) return hipSuccess;
  const dim3 grid((unsigned)g.prefix[g.count]), block(64 * kRedWaves);
  if (part_bf16 && dtype != kBF16) return hipErrorInvalidValue;  // only the bf16 matrix-core chain writes them
  switch (dtype) {
    case kF32: hipLaunchKernelGGL((bfht_reduce_grouped<float, float>), grid, block, 0, s, g); break;
    case kF16: hipLaunchKernelGGL((bfht_reduce_grouped<f16, float>), grid, block, 0, s, g); break;
    case kBF16:
      if (part_bf16) hipLaunchKernelGGL((bfht_reduce_grouped<bf16, bf16>), grid, block, 0, s, g);
      else hipLaunchKernelGGL((bfht_reduce_grouped<bf16, float>), grid, block, 0, s, g);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
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
