// Fused BlockFHTLinear forward for the reference extension's own domain
// (float32 / float16 / bfloat16, block B <= 2^14, B % in_features == 0;
// reference gate latent_weight_lab/block_fht.py:263-273, kernel
// csrc/block_fht_ext_cuda.cu:225-329) at batches of 16 tokens and more, with
// the contraction on the matrix cores.  From 256 tokens x is first re-laid out
// in MFMA operand order (launch_tile_x: one 1 KiB load per 16 tokens and step
// instead of 16 rows x 64 bytes).
//
// A workgroup owns a tile of consecutive generated blocks (32768 weights for
// 16-bit I/O, 16384 for float32; whole rows, since in_features divides B) and
// a range of tokens.  It runs the whole-block VALU generator over the tile,
// one generator call (G blocks) at a time, and the generator's final stores
// land, scaled by weight_scale and rounded to the I/O type, in an LDS table of
// 16-byte k-chunks: chunk (kc, r) = W[row0 + r][kc*CH .. kc*CH + CH - 1] at slot
// kc * pitch + mm_row(kc, r), pitch = rows + 1 (odd, so the generator's stores
// of consecutive k in one row spread over the LDS banks; the contraction reads
// 16 rows of one chunk, a permutation of 16 consecutive slots, see mm_row).
// Each wave then contracts items
// of 4 token tiles x RT row tiles (RT = 1, 2 or 4: the tile's 16-row tiles, at
// most 4):
//
//   D[t][o] = sum_k x[t][k] * W[o][k]   A = x (16 tokens x K, row-major from memory)
//                                        B = W^T (K x 16 rows, table chunks)
//
// 16-bit I/O: v_mfma_f32_16x16x32_{f16,bf16}, K = 32 per step (W rounded to
// the I/O type, as the reference's fallback rounds it before F.linear).
// float32: v_mfma_f32_16x16x4_f32, exact float32 products as the reference's
// kernel computes them; lane (l16, kq) loads x[t][16 s + 4 kq .. + 3] once and
// feeds it to four MFMAs (k order permuted alike in A and B).
// Accumulation in float32; the epilogue (lwl_bfht_linear_forward_ex) is applied
// in the stores.  The weight never touches memory.
#include "bfht_block.h"

#include <algorithm>

namespace lwl {
namespace {

typedef float f32x4m __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4m __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8m __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8m __attribute__((ext_vector_type(8)));

template <int LB, class T>
struct MmGeo {
  using Gm = Geo<LB>;
  static constexpr int EC = Gm::G * Gm::B;                             // weights per generator call
  static constexpr int TILE = sizeof(T) == 2 ? 32768 : 16384;          // weights per workgroup
  static constexpr int NC = TILE / EC;                                 // generator calls per workgroup
  static constexpr int CH = 16 / (int)sizeof(T);                       // k values per 16-byte chunk
  static constexpr int KSTEP = sizeof(T) == 2 ? 32 : 16;               // k per step (one A load per lane)
  // the table: TILE weights plus one spare chunk per k chunk (pitch = rows + 1;
  // k chunks per row <= TILE / (16 rows * CH)), plus 64 chunks that the last k
  // chunk's reads of row tiles past the tile's rows reach (an item's row tiles
  // run at most 63 rows past the table; their columns are never stored)
  static constexpr int TABLE_BYTES = TILE * (int)sizeof(T) + TILE / (16 * CH) * 16 + 64 * 16;
  static_assert(TILE % EC == 0, "whole generator calls per workgroup");
  static_assert(BlockLds<LB>::FLOATS * 4 + TABLE_BYTES <= 160 * 1024, "generator and table fit the LDS");
};

// Table row of W row r in k chunk kc.  A ds_read_b128 serves 16 lanes per LDS
// cycle over 64 banks: lanes 0-3, 12-15, 20-23, 24-27 together and 4-7, 8-11,
// 16-19, 28-31 together (the same for 32-63), i.e. rows l16 in {0-3, 12-15} of
// chunk kq = 0 with rows {4-11} of chunk 1 and the other way round (2 and 3
// alike).  Odd chunks sit pitch slots after even ones, so they hold each
// 16-row group permuted, r -> ((r ^ 1) - pitch) mod 16: every such read then
// covers the 16 16-byte bank groups once (with rows in place, pitch = 1 mod 16
// put two lanes on each of 8 groups), and a row keeps its parity, so the
// generator's stores of 8 consecutive chunks of one row still fall on 8
// distinct groups modulo 8 (the odd pitch).  The rows per tile are a multiple
// of 16, so every group is whole.
__device__ __forceinline__ int mm_row(int kc, int r, int pitch) {
  return (kc & 1) ? (r & ~15) | ((((r & 15) ^ 1) - pitch) & 15) : r;
}

// The generator's store functor: tile-relative position p = r * in + k lands in
// chunk (k / CH, r), element k % CH.
template <class T>
struct TableStore {
  T* tbl;
  int64_t base;  // first flat position of the tile
  int log_in;
  int pitch;
  float scale;
  struct Range {
    int first;
    int count;
  };
  __device__ void put(int p, float v) const {
    constexpr int CH = 16 / (int)sizeof(T);
    const int r = p >> log_in, k = p & ((1 << log_in) - 1);
    const int kc = k / CH;
    tbl[(kc * pitch + mm_row(kc, r, pitch)) * CH + (k % CH)] = from_f32<T>(v * scale);
  }
  __device__ Range range(int64_t first, int64_t count) const { return Range{(int)(first - base), (int)count}; }
  __device__ void operator()(Range rg, int i, float v) const {
    if ((unsigned)i < (unsigned)rg.count) put(rg.first + i, v);
  }
  __device__ void whole(Range rg, int b, int c, float v) const { put(rg.first + b + c, v); }
  __device__ void at(int64_t i, float v) const { put((int)(i - base), v); }
};

template <class T>
__device__ __forceinline__ f32x4m mm16(u32x4m a, u32x4m b, f32x4m c) {
  if constexpr (__is_same(T, f16))
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8m, a), __builtin_bit_cast(f16x8m, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8m, a), __builtin_bit_cast(bf16x8m, b),
                                                   c, 0, 0, 0);
}

constexpr int kMmTok = 4;    // token tiles (of 16) per item
constexpr int kMmDepth = 4;  // x prefetch distance in k steps

template <int LB, class T, int kMmRows>
__global__ __launch_bounds__(Geo<LB>::WG) void bfht_linear_small_mm(const T* __restrict__ x,
                                                                    const u32x4m* __restrict__ xt,
                                                                    const T* __restrict__ latent,
                                                                    T* __restrict__ out, int tokens, int in_f,
                                                                    int log_in, int out_f, int n, int64_t nblocks,
                                                                    uint32_t seed32, int layers, float scale,
                                                                    int token_split, LinearEpi ep) {
  using Gm = Geo<LB>;
  using MG = MmGeo<LB, T>;
  constexpr int CH = MG::CH;
  constexpr uint32_t kOff = 0x80000000u;  // buffer offset that reads 0 / drops the store
  __shared__ float smem[BlockLds<LB>::FLOATS];
  __shared__ __attribute__((aligned(16))) unsigned char table_raw[MG::TABLE_BYTES];
  T* tbl = reinterpret_cast<T*>(table_raw);
  const u32x4m* chunks = reinterpret_cast<const u32x4m*>(table_raw);
  const int64_t tile = blockIdx.x;
  const int split = blockIdx.y;
  const int64_t size = (int64_t)in_f * out_f;
  const int64_t base = tile * MG::TILE;
  const int rows_wg = MG::TILE >> log_in;  // >= 16 (host check)
  const int pitch = rows_wg + 1;

  // 1. the tile's blocks into the table (inactive slots past the last block
  //    store nothing: their rows lie past out_features and are never stored)
  for (int c = 0; c < MG::NC; ++c) {
    const int64_t slot = (tile * MG::NC + c) * Gm::G + (threadIdx.x >> Gm::LT);
    block_fwd_slot<LB, T>(latent, TableStore<T>{tbl, base, log_in, pitch, scale}, n, 0, slot, nblocks, 0, size,
                          seed32, layers, smem);
    __syncthreads();  // the generator's LDS is reused by the next call; after the last, the table is whole
  }

  // 2. items of this split: kMmTok token tiles x kMmRows row tiles, round robin over the waves
  const int row0 = (int)(base >> log_in);
  const int rows = out_f - row0 < rows_wg ? out_f - row0 : rows_wg;
  const int ntt = (tokens + 15) / 16;
  const int per_split = (ntt + token_split - 1) / token_split;
  const int tt0 = split * per_split;
  const int tt1 = tt0 + per_split < ntt ? tt0 + per_split : ntt;
  if (rows <= 0 || tt0 >= tt1) return;  // uniform across the workgroup
  const int nrt = (rows + 15) / 16;
  const int ngroups_t = (tt1 - tt0 + kMmTok - 1) / kMmTok;
  const int ngroups_r = (nrt + kMmRows - 1) / kMmRows;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int l16 = lane & 15, kq = lane >> 4;
  constexpr int kWaves = Gm::WG / 64;
  const int nsteps = in_f / MG::KSTEP;  // 64 bytes of k per step
  // x: the tiled copy (1 KiB per token tile and step, step-major) or the row-major input
  const bool tiled = xt != nullptr;
  const auto x_r = tiled ? tile_rsrc(xt, (uint64_t)ntt * nsteps * 1024) : tile_rsrc(x, (uint64_t)tokens * in_f * sizeof(T));
  const uint32_t xstride = tiled ? (uint32_t)ntt * 1024u : 64u;  // per step
  const auto o_r = tile_rsrc(out, (uint64_t)tokens * out_f * sizeof(T));
  const bool has_xs = ep.xsum != nullptr, has_base = ep.base != nullptr, has_bias = ep.bias != nullptr;
  const float cx = has_xs ? ep.cscale * *ep.coef : 0.f;
  const auto xs_r = tile_rsrc(has_xs ? (const void*)ep.xsum : (const void*)out, has_xs ? (uint64_t)tokens * 4 : 0);
  const auto b_r = tile_rsrc(has_base ? ep.base : (const void*)out, has_base ? (uint64_t)tokens * out_f * sizeof(T) : 0);
  const auto bias_r = tile_rsrc(has_bias ? ep.bias : (const void*)out, has_bias ? (uint64_t)out_f * sizeof(T) : 0);

  for (int item = wave; item < ngroups_t * ngroups_r; item += kWaves) {
    const int gt = item / ngroups_r, gr = item - gt * ngroups_r;
    const int ttb = tt0 + gt * kMmTok, rtb = gr * kMmRows;
    // x offsets of this lane's rows (tokens past the split or the batch read 0)
    uint32_t xo[kMmTok];
#pragma unroll
    for (int g = 0; g < kMmTok; ++g) {
      const int t = (ttb + g) * 16 + l16;
      if (tiled)
        xo[g] = ttb + g < tt1 ? (uint32_t)(((ttb + g) * 64 + lane) * 16) : kOff;
      else
        xo[g] = (ttb + g < tt1 && t < tokens) ? (uint32_t)(t * in_f + (MG::KSTEP / 4) * kq) * (uint32_t)sizeof(T) : kOff;
    }
    // table slot of this lane's row in row tile j, chunk 0 of step s: (4 s + kq) * pitch + 16 (rtb + j) +
    // mm_row(kq, l16) (the permutation keeps each 16-row group in place)
    const int slot0 = kq * pitch + 16 * rtb + mm_row(kq, l16, pitch);
    f32x4m acc[kMmTok][kMmRows];
#pragma unroll
    for (int g = 0; g < kMmTok; ++g)
#pragma unroll
      for (int j = 0; j < kMmRows; ++j) acc[g][j] = f32x4m{0.f, 0.f, 0.f, 0.f};
    auto xload = [&](int g, int st) -> u32x4m {  // x of token tile g at step st (past the row: 0)
      const uint32_t off = (st < nsteps && xo[g] != kOff) ? xo[g] + (uint32_t)st * xstride : kOff;
      return __builtin_amdgcn_raw_buffer_load_b128(x_r, (int)off, 0, 0);
    };
    auto step = [&](const u32x4m (&a)[kMmTok], int st) {
      u32x4m b[kMmRows];
#pragma unroll
      for (int j = 0; j < kMmRows; ++j) b[j] = chunks[slot0 + 4 * st * pitch + 16 * j];  // rows past the table: unused columns
#pragma unroll
      for (int g = 0; g < kMmTok; ++g)
#pragma unroll
        for (int j = 0; j < kMmRows; ++j) {
          if constexpr (sizeof(T) == 2) {
            acc[g][j] = mm16<T>(a[g], b[j], acc[g][j]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              acc[g][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[g][e]), __uint_as_float(b[j][e]),
                                                               acc[g][j], 0, 0, 0);
          }
        }
    };
    if (nsteps % kMmDepth == 0) {
      // x prefetched kMmDepth steps ahead into a register ring; slot d is
      // refilled right after its last use (its own registers, no copies)
      u32x4m ring[kMmDepth][kMmTok];
#pragma unroll
      for (int d = 0; d < kMmDepth; ++d) {
#pragma unroll
        for (int g = 0; g < kMmTok; ++g) ring[d][g] = xload(g, d);
      }
      for (int s0 = 0; s0 < nsteps; s0 += kMmDepth) {
#pragma unroll
        for (int d = 0; d < kMmDepth; ++d) {
          step(ring[d], s0 + d);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int g = 0; g < kMmTok; ++g) ring[d][g] = xload(g, s0 + d + kMmDepth);
        }
      }
    } else {  // one or two steps per row
      for (int st = 0; st < nsteps; ++st) {
        u32x4m a[kMmTok];
#pragma unroll
        for (int g = 0; g < kMmTok; ++g) a[g] = xload(g, st);
        step(a, st);
      }
    }
    // D[m = 4 kq + r][n = l16]: token 16 (ttb + g) + 4 kq + r, row row0 + 16 (rtb + j) + l16.
    // The epilogue's inputs of the item are loaded before its first store.
    float xs[kMmTok][4], base_v[kMmTok][kMmRows][4], bias_v[kMmRows];
    auto elem = [&](int g, int j, int r) -> int {  // element index in out, or -1
      const int t = (ttb + g) * 16 + 4 * kq + r;
      const int rr = 16 * (rtb + j) + l16;
      return (ttb + g < tt1 && t < tokens && rr < rows) ? t * out_f + row0 + rr : -1;
    };
#pragma unroll
    // (no load behind a branch on its term, which would be waited out on its
    // own: an absent term's buffer is empty and reads 0)
    for (int j = 0; j < kMmRows; ++j) bias_v[j] = buf_load<T>(bias_r, row0 + 16 * (rtb + j) + l16);
#pragma unroll
    for (int g = 0; g < kMmTok; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = (ttb + g) * 16 + 4 * kq + r;
        xs[g][r] = cx * buf_load<float>(xs_r, t < tokens ? t : -1);
#pragma unroll
        for (int j = 0; j < kMmRows; ++j) base_v[g][j][r] = buf_load<T>(b_r, elem(g, j, r));
      }
#pragma unroll
    for (int g = 0; g < kMmTok; ++g)
#pragma unroll
      for (int j = 0; j < kMmRows; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          buf_store<T>(linear_epilogue(acc[g][j][r], has_xs, xs[g][r], has_base, base_v[g][j][r], has_bias, bias_v[j]),
                       o_r, elem(g, j, r));
  }
}

template <int LB, class T>
hipError_t launch_mm_lb(const LinearArgs& a, const u32x4m* xt, hipStream_t s) {
  using Gm = Geo<LB>;
  using MG = MmGeo<LB, T>;
  const int64_t wtiles = (a.in_features * a.out_features + MG::TILE - 1) / MG::TILE;
  int log_in = 0;
  while (((int64_t)1 << log_in) < a.in_features) ++log_in;
  // row tiles per item: the tile's 16-row tiles (rows of one tile, or all of out), at most 4
  const int64_t rows = std::min<int64_t>(MG::TILE >> log_in, a.out_features);
  const int rt = rows > 32 ? 4 : rows > 16 ? 2 : 1;
#define LWL_MM(RT)                                                                                              \
  hipLaunchKernelGGL((bfht_linear_small_mm<LB, T, RT>), dim3((unsigned)wtiles, (unsigned)a.token_splits),     \
                     dim3(Gm::WG), 0, s, (const T*)a.x, xt, (const T*)a.latent, (T*)a.out, (int)a.tokens,      \
                     (int)a.in_features, log_in, (int)a.out_features, (int)a.n, a.nblocks_w, a.seed32, a.layers, \
                     a.weight_scale, a.token_splits, a.epi)
  switch (rt) {
    case 1: LWL_MM(1); break;
    case 2: LWL_MM(2); break;
    default: LWL_MM(4); break;
  }
#undef LWL_MM
  return hipGetLastError();
}

template <class T, int... LBs>
hipError_t dispatch_mm(const LinearArgs& a, const u32x4m* xt, hipStream_t s, std::integer_sequence<int, LBs...>) {
  using Fn = hipError_t (*)(const LinearArgs&, const u32x4m*, hipStream_t);
  static const Fn table[] = {&launch_mm_lb<LBs + kLinearMmMinLog, T>...};
  return table[a.log_block - kLinearMmMinLog](a, xt, s);
}

// x is read from the tiled copy from this many tokens (as the matrix-core
// kernel of block 2^15 does), while its offsets stay below 2^31.
bool mm_tiled(const LinearArgs& a) {
  const int64_t esize = a.dtype == kF32 ? 4 : 2;
  return a.tokens >= 256 && (a.tokens + 15) / 16 * (a.in_features * esize / 64) * 1024 < ((int64_t)1 << 31);
}

}  // namespace

bool linear_small_mm_applicable(const LinearArgs& a) {
  if (!linear_small_applicable(a.dtype, a.log_block, a.in_features)) return false;
  if (a.log_block < kLinearMmMinLog || a.tokens < kLinearMmMinTokens) return false;
  const int64_t tile = a.dtype == kF32 ? 16384 : 32768;
  const int64_t kstep = a.dtype == kF32 ? 16 : 32;
  // whole k steps, and at least one 16-row tile per workgroup (the table's k
  // chunks per row then fit its spare chunks)
  return a.in_features % kstep == 0 && tile / a.in_features >= 16;
}

size_t linear_small_mm_workspace_bytes(const LinearArgs& a) {
  if (!linear_small_mm_applicable(a) || !mm_tiled(a)) return 0;
  const int64_t esize = a.dtype == kF32 ? 4 : 2;
  return (size_t)((a.tokens + 15) / 16) * (size_t)(a.in_features * esize / 64) * 1024;
}

int linear_small_mm_token_splits(const LinearArgs& a) {
  // Each split regenerates its tile (the VALU generator takes ~15 us per 2^14
  // weights on one CU, as long as the contraction of ~1000 tokens), and one
  // workgroup fills a CU's LDS: about one workgroup per CU, at least 64 tokens
  // per split.
  const int64_t tile = a.dtype == kF32 ? 16384 : 32768;
  const int64_t wtiles = (a.in_features * a.out_features + tile - 1) / tile;
  int64_t split = (256 + wtiles - 1) / wtiles;
  const int64_t most = (a.tokens + 63) / 64;
  if (split > most) split = most;
  if (split > 65535) split = 65535;
  return (int)(split < 1 ? 1 : split);
}

hipError_t launch_linear_small_mm(const LinearArgs& a, hipStream_t s) {
  using Seq = std::make_integer_sequence<int, kLinearSmallMaxLog - kLinearMmMinLog + 1>;
  const u32x4m* xt = nullptr;
  if (mm_tiled(a)) {  // the tiled copy fills the start of the workspace
    const int64_t esize = a.dtype == kF32 ? 4 : 2;
    const hipError_t e = launch_tile_x(a.x, a.work, a.tokens, a.in_features * esize, s);
    if (e != hipSuccess) return e;
    xt = (const u32x4m*)a.work;
  }
  switch (a.dtype) {
    case kF32: return dispatch_mm<float>(a, xt, s, Seq{});
    case kF16: return dispatch_mm<f16>(a, xt, s, Seq{});
    case kBF16: return dispatch_mm<bf16>(a, xt, s, Seq{});
  }
  return hipErrorInvalidValue;
}

}  // namespace lwl
