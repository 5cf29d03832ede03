// BlockFHT generator kernels at block size 2^15 on the matrix cores: forward
// (signed bf16 output slice) and backward (float32 per-block partial latent
// gradients).  The chain itself (layouts, Walsh stages, LDS exchanges, sign
// words) is in bfht_mfma_chain.h.
//
// Reference semantics: latent_weight_lab/block_fht.py:84-109 (forward) and
// csrc/block_fht_ext_cuda.cu:185-223 (backward: the same chain with the sign
// layers in reverse order).
#include "bfht_mfma_chain.h"

namespace lwl {
namespace mfma15 {
namespace {

// ---------------------------------------------------------------- forward

// The 16 bytes that start M bf16 elements before chunk b: the last M elements
// of chunk a followed by the first 8 - M of b (bytes 16 - 2M .. 31 - 2M of a:b).
template <int M>
__device__ __forceinline__ u32x4 chunk_shifted(const u32x4& a, const u32x4& b) {
  const uint32_t w[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  constexpr int o = 16 - 2 * M, q = o >> 2, r = o & 3;
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (r == 0) v[i] = w[q + i];
    else v[i] = __builtin_amdgcn_alignbyte(w[q + i + 1], w[q + i], r);
  }
  return v;
}

// Stores block positions [lo, hi) of a staged block to oblk (2-byte aligned,
// M = its element offset from a 16-byte boundary): slot j of the aligned grid
// holds positions 8j - M .. 8j - M + 7, built from staged chunks j - 1 and j.
// Slots inside [lo, hi) take one 16-byte store; the slots at the range's ends,
// shared with other blocks' outputs, get element stores of their positions in
// the range.  Slots j = 0 .. kChunks (the last one only exists for M > 0).
template <int M>
__device__ __forceinline__ void store_range_shifted(const u32x4* stage, __bf16* oblk, int lo, int hi) {
  const auto a_r = rsrc(oblk - M, (uint32_t)((kChunks + 1) * 16));
  uint16_t* o16 = reinterpret_cast<uint16_t*>(oblk);
  constexpr int kPer = kChunks / kThreads;
#pragma unroll
  for (int i = 0; i <= kPer; ++i) {
    const int j = i * kThreads + (int)threadIdx.x;
    const int p0 = 8 * j - M;
    if (j > kChunks || p0 + 8 <= lo || p0 >= hi) continue;
    const u32x4 a = stage[stage_slot(j > 0 ? j - 1 : 0)];
    const u32x4 b = stage[stage_slot(j < kChunks ? j : kChunks - 1)];
    if (p0 >= lo && p0 + 8 <= hi) {
      __builtin_amdgcn_raw_buffer_store_b128(chunk_shifted<M>(a, b), a_r, j * 16, 0, kStreamStore);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int p = p0 + e;  // chunk j - 1 for e < M, chunk j from e = M
        if (p >= lo && p < hi) {
          const u32x4& c = e < M ? a : b;
          const int q = (e - M) & 7;
          o16[p] = (uint16_t)(c[q >> 1] >> (16 * (q & 1)));
        }
      }
    }
  }
}

template <int L, bool kWhole>
__global__ __launch_bounds__(kThreads) void bfht_mfma15_fwd(const __bf16* __restrict__ latent,
                                                            __bf16* __restrict__ out, int n,
                                                            int64_t first_block, int64_t start,
                                                            int64_t stop, uint32_t seed32) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kChainLdsBytes];
  const int64_t block = first_block + blockIdx.x;
  const Ctx x = make_ctx(seed32, block);
  u32x4 src[kTiles][2];
  load_latent<kWhole>(x, latent, n, src);
  f32x16 acc[kTiles];
  uint32_t nw[4];
  // block-local output range [lo, hi); out element of block position p is (base - start) + p
  const int64_t base = block * kB;
  const int lo = kWhole ? 0 : (int)(start - base > 0 ? start - base : 0);
  const int hi = kWhole ? kB : (int)(stop - base < kB ? stop - base : kB);
  __bf16* oblk = out + (base - start);
  const bool full = kWhole || (lo == 0 && hi == kB && (((uintptr_t)oblk & 15) == 0));
  if constexpr (L % 2 == 1) {
    // a whole block (uniform): the chain ends in layout F and each lane stores
    // its chunks directly
    if (full) {
      run_chain<L, true>(acc, x, lds, src, [](int i) { return i; }, nw);
      store_direct(acc, x, reinterpret_cast<const uint32_t*>(lds + kLdsBytes) + (L - 1) * kWordsPerLayer,
                   rsrc(oblk, (uint32_t)(kB * 2)));
      return;
    }
  }
  run_chain<L>(acc, x, lds, src, [](int i) { return i; }, nw);
  // The signed bf16 block goes through the free exchange buffer in position
  // order, then to memory with consecutive threads on consecutive chunks.
  u32x4* stage = reinterpret_cast<u32x4*>(lds + (L & 1) * kXBufBytes);
  stage_output<L>(acc, nw, x, stage);
  __syncthreads();
  if (!kWhole && !full && (((uintptr_t)oblk & 1) == 0)) {
    // part of a block, or an output off the 16-byte grid: 16-byte stores on the
    // grid, element stores at the range's ends (uniform branch)
    switch (((uintptr_t)oblk >> 1) & 7) {
      case 0: store_range_shifted<0>(stage, oblk, lo, hi); break;
      case 1: store_range_shifted<1>(stage, oblk, lo, hi); break;
      case 2: store_range_shifted<2>(stage, oblk, lo, hi); break;
      case 3: store_range_shifted<3>(stage, oblk, lo, hi); break;
      case 4: store_range_shifted<4>(stage, oblk, lo, hi); break;
      case 5: store_range_shifted<5>(stage, oblk, lo, hi); break;
      case 6: store_range_shifted<6>(stage, oblk, lo, hi); break;
      default: store_range_shifted<7>(stage, oblk, lo, hi); break;
    }
    return;
  }
  const auto out_r = rsrc(full ? (const void*)oblk : (const void*)out, full ? (uint32_t)(kB * 2) : 0u);
  uint16_t* oblk16 = reinterpret_cast<uint16_t*>(oblk);
  constexpr int kPer = kChunks / kThreads;
  u32x4 v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = i * kThreads + (int)threadIdx.x;
    v[i] = stage[stage_slot(c)];
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int p = (i * kThreads + (int)threadIdx.x) * 8;
    if (full) {
      __builtin_amdgcn_raw_buffer_store_b128(v[i], out_r, p * 2, 0, kStreamStore);
    } else if (p + 8 > lo && p < hi) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (p + e >= lo && p + e < hi) oblk16[p + e] = (uint16_t)(v[i][e >> 1] >> (16 * (e & 1)));
    }
  }
}

// ---------------------------------------------------------------- backward

// Loads block positions [lo, hi) of a block's gradient that starts M elements
// past a 16-byte boundary (gblk, 2-byte aligned), zero elsewhere: the chunk at
// positions p .. p + 7 is elements M .. 7 of aligned slot p / 8 followed by
// elements 0 .. M - 1 of the next slot.  A slot is read only when it holds
// positions of the range; the buffer spans the gradient's 16-byte granules
// (from the one holding its first element to the one holding its last, gend
// is one past it; at most the block's kChunks + 1 slots), so no read leaves
// them, and positions outside the range read from those granules are zeroed.
template <int M>
__device__ __forceinline__ void load_grad_shifted(const Ctx& x, const __bf16* gblk, const __bf16* gend, int lo,
                                                  int hi, u32x4 (&src)[kTiles][2]) {
  const uintptr_t a0 = (uintptr_t)gblk - 2 * M;
  const uintptr_t a1 = ((uintptr_t)gend + 15) & ~(uintptr_t)15;
  // every slot of the block lies in the first kChunks + 1 slots from a0
  const uintptr_t span = a1 - a0 < (uintptr_t)(kChunks + 1) * 16 ? a1 - a0 : (uintptr_t)(kChunks + 1) * 16;
  const auto g_r = rsrc((const void*)a0, (uint32_t)span);
  constexpr uint32_t kOff = 0x80000000u;
  load_source(
      x,
      [&](int p) -> u32x4 {
        const bool use_a = p + 7 - M >= lo && p < hi;            // slot p/8: positions p .. p + 7 - M
        const bool use_b = M > 0 && p + 7 >= lo && p + 8 - M < hi;  // next slot: p + 8 - M .. p + 7
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(g_r, (int)(use_a ? (uint32_t)(2 * p) : kOff), 0, 0);
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(g_r, (int)(use_b ? (uint32_t)(2 * p + 16) : kOff), 0, 0);
        u32x4 v = chunk_shifted<8 - M>(a, b);
        if (p < lo || p + 8 > hi) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (p + e < lo || p + e >= hi) v[e >> 1] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
        }
        return v;
      },
      src);
}

// Per-block partial latent gradient (first n positions) of the
// adjoint chain D_0 H D_1 ... H D_L applied to grad scattered into the block.
// The rows are bfloat16 (the gradient's own type; each of the ~2^8 terms of a
// position's sum carries one bf16 rounding, ~2^-9 relative, and the sum is
// formed in float32), half the traffic of float32 rows in both kernels.
// kWhole: every block's gradient is read whole from a 16-byte aligned place
// and n % 8 == 0 (the launcher checks), so no partial-chunk paths are needed.
template <int L, bool kWhole>
__global__ __launch_bounds__(kThreads) void bfht_mfma15_bwd(const __bf16* __restrict__ grad,
                                                            __bf16* __restrict__ partial, int n,
                                                            int64_t first_block, int64_t start,
                                                            int64_t stop, uint32_t seed32) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kChainLdsBytes];
  const int64_t slot = blockIdx.x;
  const int64_t block = first_block + slot;
  const Ctx x = make_ctx(seed32, block);
  const int64_t base = block * kB;
  const int lo = kWhole ? 0 : (int)(start - base > 0 ? start - base : 0);
  const int hi = kWhole ? kB : (int)(stop - base < kB ? stop - base : kB);
  const __bf16* gblk = grad + (base - start);
  const bool full = kWhole || (lo == 0 && hi == kB && (((uintptr_t)gblk & 15) == 0));
  const auto g_r = rsrc(full ? (const void*)gblk : (const void*)grad, full ? (uint32_t)(kB * 2) : 0u);
  const uint16_t* gblk16 = reinterpret_cast<const uint16_t*>(gblk);
  u32x4 src[kTiles][2];
  if (!full && (((uintptr_t)gblk & 1) == 0)) {
    // part of a block, or a gradient off the 16-byte grid: aligned 16-byte slot loads (uniform branch)
    const __bf16* gend = grad + (stop - start);
    switch (((uintptr_t)gblk >> 1) & 7) {
      case 0: load_grad_shifted<0>(x, gblk, gend, lo, hi, src); break;
      case 1: load_grad_shifted<1>(x, gblk, gend, lo, hi, src); break;
      case 2: load_grad_shifted<2>(x, gblk, gend, lo, hi, src); break;
      case 3: load_grad_shifted<3>(x, gblk, gend, lo, hi, src); break;
      case 4: load_grad_shifted<4>(x, gblk, gend, lo, hi, src); break;
      case 5: load_grad_shifted<5>(x, gblk, gend, lo, hi, src); break;
      case 6: load_grad_shifted<6>(x, gblk, gend, lo, hi, src); break;
      default: load_grad_shifted<7>(x, gblk, gend, lo, hi, src); break;
    }
  } else {
    load_source(
        x,
        [&](int p) -> u32x4 {
          if (full) return __builtin_amdgcn_raw_buffer_load_b128(g_r, p * 2, 0, 0);
          u32x4 v = {0u, 0u, 0u, 0u};
          if (p + 8 > lo && p < hi) {
  #pragma unroll
            for (int e = 0; e < 8; ++e)
              if (p + e >= lo && p + e < hi) v[e >> 1] |= (uint32_t)gblk16[p + e] << (16 * (e & 1));
          }
          return v;
        },
        src);
  }
  f32x16 acc[kTiles];
  uint32_t nw[4];
  __bf16* row = partial + slot * mfma15_part_stride(n);
  if constexpr (L % 2 == 1) {
    // odd L: the chain ends in layout F and the row goes out from registers,
    // as the forward's whole blocks do, in whole 16-byte chunks up to the row
    // stride (n rounded up to 8; the block sum reads only the first n)
    run_chain<L, true>(acc, x, lds, src, [](int i) { return L - i; }, nw);
    store_direct(acc, x, reinterpret_cast<const uint32_t*>(lds + kLdsBytes) + (L - 1) * kWordsPerLayer,
                 rsrc(row, (uint32_t)mfma15_part_stride(n) * 2u));
    return;
  }
  run_chain<L>(acc, x, lds, src, [](int i) { return L - i; }, nw);
  write_partial_row<L, kWhole, __bf16>(acc, nw, x, lds, row, n, 1.0f);
}

// ---------------------------------------------------------------- grouped


// Whole weight of each job (positions [0, size)): the chain of bfht_mfma15_fwd,
// the bf16 output times the job's weight scale.
template <int L>
__global__ __launch_bounds__(kThreads) void bfht_mfma15_fwd_grouped(const GroupTable g) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kChainLdsBytes];
  const int j = group_job(g, (int)blockIdx.x);
  const GroupJob& jb = g.job[j];
  const int64_t block = (int64_t)blockIdx.x - g.prefix[j];
  const Ctx x = make_ctx(jb.seed32, block);
  u32x4 src[kTiles][2];
  load_latent(x, static_cast<const __bf16*>(jb.src), jb.n, src);
  f32x16 acc[kTiles];
  uint32_t nw[4];
  const int64_t base = block * kB;
  const int hi = jb.size - base < kB ? (int)(jb.size - base) : kB;
  __bf16* oblk = static_cast<__bf16*>(jb.dst) + base;
  const bool full = hi == kB && (((uintptr_t)oblk & 15) == 0);
  if constexpr (L % 2 == 1) {
    // a whole block (uniform): layout F, direct stores, as bfht_mfma15_fwd
    if (full) {
      run_chain<L, true>(acc, x, lds, src, [](int i) { return i; }, nw);
      store_direct(acc, x, reinterpret_cast<const uint32_t*>(lds + kLdsBytes) + (L - 1) * kWordsPerLayer,
                   rsrc(oblk, (uint32_t)(kB * 2)), jb.scale);
      return;
    }
  }
  run_chain<L>(acc, x, lds, src, [](int i) { return i; }, nw);
  u32x4* stage = reinterpret_cast<u32x4*>(lds + (L & 1) * kXBufBytes);
  stage_output<L>(acc, nw, x, stage);
  __syncthreads();
  const auto out_r = rsrc(full ? (const void*)oblk : jb.dst, full ? (uint32_t)(kB * 2) : 0u);
  uint16_t* oblk16 = reinterpret_cast<uint16_t*>(oblk);
  const float scale = jb.scale;
  constexpr int kPer = kChunks / kThreads;
  u32x4 v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = i * kThreads + (int)threadIdx.x;
    v[i] = stage[stage_slot(c)];
    if (scale != 1.0f) v[i] = scale_chunk(v[i], scale);
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int p = (i * kThreads + (int)threadIdx.x) * 8;
    if (full) {
      __builtin_amdgcn_raw_buffer_store_b128(v[i], out_r, p * 2, 0, kStreamStore);
    } else if (p < hi) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (p + e < hi) oblk16[p + e] = (uint16_t)(v[i][e >> 1] >> (16 * (e & 1)));
    }
  }
}

// Per-block partial rows of each job's whole-weight gradient (bf16 weight
// gradient, as bfht_mfma15_bwd), into the job's partial rows.
template <int L>
__global__ __launch_bounds__(kThreads) void bfht_mfma15_bwd_grouped(const GroupTable g) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kChainLdsBytes];
  const int j = group_job(g, (int)blockIdx.x);
  const GroupJob& jb = g.job[j];
  const int64_t slot = (int64_t)blockIdx.x - g.prefix[j];
  const Ctx x = make_ctx(jb.seed32, slot);
  const int64_t base = slot * kB;
  const int hi = jb.size - base < kB ? (int)(jb.size - base) : kB;
  const __bf16* gblk = static_cast<const __bf16*>(jb.src) + base;
  const bool full = hi == kB && (((uintptr_t)gblk & 15) == 0);
  const auto g_r = rsrc(full ? (const void*)gblk : jb.src, full ? (uint32_t)(kB * 2) : 0u);
  const uint16_t* gblk16 = reinterpret_cast<const uint16_t*>(gblk);
  u32x4 src[kTiles][2];
  if (!full && (((uintptr_t)gblk & 1) == 0)) {
    // the last, partial block, or a weight gradient off the 16-byte grid (uniform branch)
    const __bf16* gend = static_cast<const __bf16*>(jb.src) + jb.size;
    switch (((uintptr_t)gblk >> 1) & 7) {
      case 0: load_grad_shifted<0>(x, gblk, gend, 0, hi, src); break;
      case 1: load_grad_shifted<1>(x, gblk, gend, 0, hi, src); break;
      case 2: load_grad_shifted<2>(x, gblk, gend, 0, hi, src); break;
      case 3: load_grad_shifted<3>(x, gblk, gend, 0, hi, src); break;
      case 4: load_grad_shifted<4>(x, gblk, gend, 0, hi, src); break;
      case 5: load_grad_shifted<5>(x, gblk, gend, 0, hi, src); break;
      case 6: load_grad_shifted<6>(x, gblk, gend, 0, hi, src); break;
      default: load_grad_shifted<7>(x, gblk, gend, 0, hi, src); break;
    }
  } else {
    load_source(
        x,
        [&](int p) -> u32x4 {
          if (full) return __builtin_amdgcn_raw_buffer_load_b128(g_r, p * 2, 0, 0);
          u32x4 v = {0u, 0u, 0u, 0u};
          if (p < hi) {
  #pragma unroll
            for (int e = 0; e < 8; ++e)
              if (p + e < hi) v[e >> 1] |= (uint32_t)gblk16[p + e] << (16 * (e & 1));
          }
          return v;
        },
        src);
  }
  f32x16 acc[kTiles];
  uint32_t nw[4];
  __bf16* row = static_cast<__bf16*>(jb.part) + slot * (int64_t)jb.stride;
  if constexpr (L % 2 == 1) {
    // odd L: the row from layout F in whole 16-byte chunks up to the row stride
    // (a multiple of 64; the block sum reads only the first n), as bfht_mfma15_bwd
    run_chain<L, true>(acc, x, lds, src, [](int i) { return L - i; }, nw);
    store_direct(acc, x, reinterpret_cast<const uint32_t*>(lds + kLdsBytes) + (L - 1) * kWordsPerLayer,
                 rsrc(row, (uint32_t)jb.stride * 2u));
    return;
  }
  run_chain<L>(acc, x, lds, src, [](int i) { return L - i; }, nw);
  write_partial_row<L, false, __bf16>(acc, nw, x, lds, row, jb.n, 1.0f);
}

}  // namespace
}  // namespace mfma15

bool mfma15_applicable(const BfhtArgs& a, bool fwd) {
  // 16-byte vector loads of the latent and stores of the partial rows need
  // aligned bases; the backward reads the gradient in aligned 16-byte slots
  // whatever its offset, and output alignment is handled per block.
  const bool aligned = ((uintptr_t)a.src % (fwd ? 16 : 2) == 0) &&
                       (a.work == nullptr || (uintptr_t)a.work % 16 == 0);
  return a.dtype == kBF16 && a.log_block == mfma15::kLog && a.nblocks > 0 && a.n <= mfma15::kB && aligned;
}

namespace {

template <bool kWhole>
hipError_t launch_mfma15_shape(const BfhtArgs& a, hipStream_t s, bool fwd) {
  using namespace mfma15;
  const dim3 grid((unsigned)a.nblocks), block(kThreads);
  auto* src = (const __bf16*)a.src;
  const int n = (int)a.n;
  if (fwd) {
    auto* dst = (__bf16*)a.dst;
    switch (a.layers) {
      case 1: hipLaunchKernelGGL((bfht_mfma15_fwd<1, kWhole>), grid, block, 0, s, src, dst, n, a.first_block, a.start, a.stop, a.seed32); break;
      case 2: hipLaunchKernelGGL((bfht_mfma15_fwd<2, kWhole>), grid, block, 0, s, src, dst, n, a.first_block, a.start, a.stop, a.seed32); break;
      case 3: hipLaunchKernelGGL((bfht_mfma15_fwd<3, kWhole>), grid, block, 0, s, src, dst, n, a.first_block, a.start, a.stop, a.seed32); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  auto* part = (__bf16*)a.work;  // bf16 partial rows (summed in float32, bfht_reduce_blocks)
  switch (a.layers) {
    case 1: hipLaunchKernelGGL((bfht_mfma15_bwd<1, kWhole>), grid, block, 0, s, src, part, n, a.first_block, a.start, a.stop, a.seed32); break;
    case 2: hipLaunchKernelGGL((bfht_mfma15_bwd<2, kWhole>), grid, block, 0, s, src, part, n, a.first_block, a.start, a.stop, a.seed32); break;
    case 3: hipLaunchKernelGGL((bfht_mfma15_bwd<3, kWhole>), grid, block, 0, s, src, part, n, a.first_block, a.start, a.stop, a.seed32); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_mfma15_grouped(const GroupTable& g, int layers, hipStream_t s, bool fwd) {
  using namespace mfma15;
  if (g.count <= 0 || g.prefix[g.count] == 0) return hipSuccess;
  const dim3 grid((unsigned)g.prefix[g.count]), block(kThreads);
#define LWL_GROUPED(L)                                                       \
  if (fwd)                                                                   \
    hipLaunchKernelGGL((bfht_mfma15_fwd_grouped<L>), grid, block, 0, s, g); \
  else                                                                       \
    hipLaunchKernelGGL((bfht_mfma15_bwd_grouped<L>), grid, block, 0, s, g)
  switch (layers) {
    case 1: LWL_GROUPED(1); break;
    case 2: LWL_GROUPED(2); break;
    case 3: LWL_GROUPED(3); break;
    default: return hipErrorInvalidValue;
  }
#undef LWL_GROUPED
  return hipGetLastError();
}

hipError_t launch_mfma15(const BfhtArgs& a, hipStream_t s, bool fwd) {
  using namespace mfma15;
  // whole blocks: [start, stop) covers exactly blocks first_block .. +nblocks, and the
  // slice base (out / grad) is 16-byte aligned, so every block's base is too
  const bool whole = a.start == a.first_block * kB && a.stop == (a.first_block + a.nblocks) * kB &&
                     (uintptr_t)a.dst % 16 == 0 && (uintptr_t)a.src % 16 == 0 && a.n % 8 == 0;
  return whole ? launch_mfma15_shape<true>(a, s, fwd) : launch_mfma15_shape<false>(a, s, fwd);
}

}  // namespace lwl
