// Fused BlockFHTLinear forward: out = weight_scale * x @ W^T with W generated
// on chip, block by block, and contracted there (three-block tiles, below, are
// the exception: each workgroup parks part of its tiles in its own workspace).
//
// W[o, i] = y[o * in + i] where y is the BlockFHT output of the latent over
// size = in * out (reference latent_weight_lab/block_fht.py:251-288).  One
// workgroup owns one generated block b (2^15 weights, the matrix-core chain of
// bfht_mfma_chain.h) and one range of tokens: it generates the block into LDS
// as bf16, then contracts it with its tokens' rows of x on v_mfma_f32_16x16x32_bf16:
//
//   D[t][o] = sum_k x[t][k] * W[o][k]     A = x tile (16 tokens x 32 k, from memory)
//                                          B = W^T tile (32 k x 16 rows, from LDS)
//
// Block b covers flat positions [b*B, (b+1)*B): rows o_first .. o_last.  A row
// whose positions start in an earlier block or end in a later one is partial:
// its float32 partial dot products go to the workspace, and a second kernel
// adds the two halves of each straddling row (two terms: the sum does not
// depend on the order).  Rows inside the block are written directly.
//
// x is read as MFMA A operands: per k step, lane (l16, kq) holds the 8 values
// k = 32*step + 8*kq .. +7 of token 16*tile + l16.  Read in place from the
// row-major [tokens, in] input, one such load touches 16 rows x 64 bytes, and
// every generated block re-reads all of x, so for large batches x is first
// re-laid out (bfht_linear_tile_x) so that each load reads 1 KiB contiguous.
//
// Reference kernel: csrc/block_fht_ext_cuda.cu:225-329 (which regenerates each
// block per 8-token tile and requires block_size % in_features == 0).
#include "bfht_mfma_chain.h"

#include <algorithm>
#include <climits>
#include <type_traits>
#include <vector>

namespace lwl {
namespace {

using namespace mfma15;

typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kTokTile = 16;  // tokens per MFMA tile
constexpr int kXcds = 8;      // MI355X: workgroup i is dispatched to XCD i % 8
constexpr int kKStep = 32;    // k per MFMA
constexpr int kGroup = 4;     // token tiles per wave pass (each W read feeds kGroup MFMAs)
constexpr int kDepth = 4;     // x prefetch distance in k steps (and nsteps' rounding)
constexpr int kDepthSingle = 12;  // the same for single-tile passes (decode: one token tile per workgroup)

// Scattered bf16 store written through the XCD's L2 (sc0 sc1).  The combine
// kernel's stores touch one 2-byte element per 128-byte line; written back,
// each such line would be a partial-line write-back at the kernel's end.
__device__ __forceinline__ void store_bf16_through(__bf16* p, float v) {
  const uint32_t bits = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v);
  asm volatile("global_store_short %0, %1, off sc0 sc1" ::"v"(p), "v"(bits) : "memory");
}

// The bf16 at byte offset `off` of a buffer, as float (0 past its end).
__device__ __forceinline__ float bf16_at(__amdgpu_buffer_rsrc_t r, int off) {
  const uint16_t h = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  return (float)__builtin_bit_cast(__bf16, h);
}

__device__ __forceinline__ f32x4v mfma16(u32x4 a, u32x4 b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// A workgroup contracts a tile of KB consecutive generated blocks (KB = 1, or 2
// for large batches: twice the rows per loaded x element, half the x traffic).
// Up to kMaxNT tiles of 16 output rows per block (in_features >= 2^15/(16*kMaxNT - 2)), and the
// k-major table (4*linear_steps(in) chunks x `pitch` rows x 16 bytes) must fit in the
// workgroup's LDS (all 160 KiB of a gfx950 CU; the generator's exchange uses the first 128).
// Together: in_features % 8 == 0 and 528 <= in_features <= 5120.
constexpr int kMaxNT = 4;
constexpr int kLinearMaxIn = 5120;  // the range the tests cover (the table itself would fit larger rows)
constexpr int kMaxNT2 = 6;  // two blocks per workgroup: 16-row tiles (register budget)
constexpr int kLinearLdsBytes = 160 * 1024;
static_assert(kLinearLdsBytes >= kChainLdsBytes && kLinearLdsBytes >= kChain2LdsBytes,
              "the generator chains run in the same LDS");

// output rows a tile of kb blocks can touch, incl. the two partial ones
__host__ __device__ constexpr int64_t linear_rows(int64_t in_features, int kb) {
  return ((int64_t)kb * kB + in_features - 1) / in_features + 1;
}
__host__ __device__ constexpr int64_t linear_row_tiles(int64_t in_features, int kb = 1) {
  return (linear_rows(in_features, kb) + 15) / 16;
}

// k steps of 32 per row, rounded up to whole prefetch rounds of kDepth steps
__host__ __device__ constexpr int linear_steps(int64_t in_features) {
  return (int)(((in_features + kKStep - 1) / kKStep + kDepth - 1) / kDepth * kDepth);
}

// Table chunk (kc, r) — row r of the tile, k chunk kc — lives at
// kc * pitch + table_row(kc, r) + (kc >> 2): every k step's 4 chunks are
// shifted one slot further than the previous step's.  That makes the scatter
// of a generated block conflict-free: a ds_write_b128 serves 8 consecutive
// lanes per LDS cycle over 32 banks, and the lanes of one scatter write hold
// chunks 4 apart in one row (kc, kc + 4, ... — one parity, so one row
// position), whose slots then differ by 4 * pitch + 1, an odd number, so they
// fall in 8 distinct 16-byte bank groups for any pitch.  The contraction reads
// one step's chunks at a common shift: lane (l16, kq) reads row 16 nt + l16 of
// chunk 4 step + kq.  A ds_read_b128 serves 16 lanes per cycle over 64 banks,
// lanes 0-3, 12-15, 20-23, 24-27 together and 4-7, 8-11, 16-19, 28-31 together
// (the same for 32-63), i.e. rows l16 in {0-3, 12-15} of chunk kq = 0 with
// rows {4-11} of chunk 1 and the other way round (2 and 3 alike); odd chunks
// sit pitch slots after even ones, so they hold each whole 16-row group
// permuted, r -> ((r ^ 1) - pitch) mod 16, and every read covers the 16 bank
// groups once (with rows in place, an exact pitch of 23 rows put two lanes on
// each of 8 groups: 1204 conflict cycles per wave at in_features 3072).
__host__ __device__ constexpr int table_row(int kc, int r, int pitch) {
  return ((kc & 1) && r < (pitch & ~15)) ? (r & ~15) | ((((r & 15) ^ 1) - pitch) & 15) : r;
}
__device__ __forceinline__ int table_slot(int kc, int r, int pitch) {
  return kc * pitch + table_row(kc, r, pitch) + (kc >> 2);
}

constexpr int64_t linear_table_bytes(int64_t in_features, int64_t pitch) {
  const int64_t steps = linear_steps(in_features);
  return (4 * steps * pitch + steps) * 16;
}
// Three-block row tiles: the first k steps whose table (4 pitch + 1 slots per
// step) fits in the LDS, in whole prefetch rounds; the W tiles of the steps
// after them go to the workgroup's overflow in global memory.
__host__ __device__ constexpr int linear_lds_steps(int nsteps, int pitch) {
  const int fit = (kLinearLdsBytes / 16) / (4 * pitch + 1) / kDepth * kDepth;
  return fit < nsteps ? fit : nsteps;
}
// Three-block row tiles: the staging area of the first block's generated
// chunks (8 per thread) while the other two blocks' chains run.
constexpr int kStageBytes = 8 * mfma15::kThreads * 16;
// Table rows: whole 16-row tiles when they fit in the LDS, else the exact row
// count (the reads of the last row tile then run up to 15 rows past the table,
// into entries whose output columns are never stored, so an exact table leaves
// that much LDS free).
constexpr int64_t kExactPitchSlack = 16 * 16;
int linear_pitch(int64_t in_features, int kb) {
  const int64_t padded = 16 * linear_row_tiles(in_features, kb);
  return (int)(linear_table_bytes(in_features, padded) <= kLinearLdsBytes ? padded : linear_rows(in_features, kb));
}
bool linear_pitch_fits(int64_t in_features, int kb) {
  const int pitch = linear_pitch(in_features, kb);
  const bool exact = pitch < 16 * linear_row_tiles(in_features, kb);
  return linear_table_bytes(in_features, pitch) + (exact ? kExactPitchSlack : 0) <= kLinearLdsBytes;
}

// Batches from this many tokens read x from the tiled copy.
constexpr int64_t kTiledMinTokens = 256;

// Tiled x: for token tile T (16 tokens) and k step s, 64 16-byte chunks in
// lane order, chunk (l16 + 16*kq) = x[16*T + l16][32*s + 8*kq .. +7]; tokens
// past the end and k past the row are zero.  Step-major: the 1 KiB group of
// (s, T) is the (s * tiles + T)-th, so the token tiles a workgroup reads at one
// k step are one contiguous run (token-tile-major, they lay a whole row's
// steps apart and the contraction's x stream ran slower).
struct XTiling {
  int64_t tiles;  // token tiles
  int steps;      // k steps holding data: ceil(in / 32)
  size_t bytes() const { return (size_t)tiles * (size_t)steps * 1024; }
};

XTiling x_tiling(const LinearArgs& a) {
  return XTiling{(a.tokens + kTokTile - 1) / kTokTile, (int)((a.in_features + kKStep - 1) / kKStep)};
}

// buffer offsets into the tiled copy stay below 2^31 (the out-of-range voffset is 2^31)
bool linear_tiled(const LinearArgs& a) {
  return a.tokens >= kTiledMinTokens && x_tiling(a).bytes() < ((size_t)1 << 31);
}

// Rows of a three-block row tile at this row length, or 0: three blocks hold a
// whole number of rows that two do not, in one or two 16-row tiles, with no k
// padding (in_features 3072: 32 rows).
int linear_three_block_rows(int64_t in_features) {
  const int64_t len = 3 * (int64_t)mfma15::kB;
  if (in_features % (kKStep * kDepth) != 0 || len % in_features != 0 || (2 * mfma15::kB) % in_features == 0)
    return 0;
  const int64_t rows = len / in_features;
  return rows % 16 == 0 && rows / 16 <= 2 ? (int)rows : 0;
}

// Batches from this many tokens use three-block tiles where they apply: a
// workgroup's generation (one chain, the staging round trip, the pair chain,
// the scatter) takes ~22 us against the pair chain's ~13, and the contraction
// streams a third less x (3072 -> 768, three / two blocks: 48.8 / 43.1 us at
// 1536 tokens, 51.5 / 52.8 at 2048, 51.7 / 57.8 at 2560, 66.0 / 77.0 at 4096,
// 189 / 237 at 16384).
constexpr int64_t kThreeBlockMinTokens = 2048;

size_t partial_bytes(const LinearArgs& a) {
  if (a.blocks_per_wg == 3) {  // every work item's overflow W tiles and staging area
    const int nt = a.rows_per_tile / 16, nsteps = linear_steps(a.in_features);
    const int64_t per_item = (int64_t)(nsteps - linear_lds_steps(nsteps, 16 * nt)) * nt * 1024 + kStageBytes;
    const int64_t items = (a.out_features + a.rows_per_tile - 1) / a.rows_per_tile * a.token_splits;
    return ((size_t)(items * per_item) + 255) / 256 * 256;
  }
  if (a.rows_per_tile > 0) return 0;  // row tiles: no straddling rows
  const int64_t ntiles = (a.nblocks_w + a.blocks_per_wg - 1) / a.blocks_per_wg;
  return ((size_t)ntiles * 2 * (size_t)a.tokens * sizeof(float) + 255) / 256 * 256;
}

// One wave per (token tile T, run of kTileSteps k steps): lane l reads the
// 16 bytes at byte 64 s + 16 (l >> 4) of row 16 T + (l & 15) for every step s of
// the run (all loads in flight before the first store; each pair of steps reads
// 16 whole 128-byte row segments) and writes the 1 KiB chunk group of each
// step: the MFMA A operands of 16 tokens x 64 bytes of k (32 bf16 / f16 values,
// or 16 float32).  The copy is stored write-through: the fused kernel reads it
// from other XCDs, and streaming it out during the kernel avoids a serial L2
// write-back at its end.
constexpr int kTileSteps = 8;

__global__ __launch_bounds__(256) void bfht_linear_tile_x(const unsigned char* __restrict__ x, u32x4* __restrict__ xt,
                                                          int tokens, int row_bytes, int steps, int runs, int waves) {
  const int wv = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // scalar: uniform resources
  if (wv >= waves) return;
  const int tt = wv / runs;
  const int s0 = (wv - tt * runs) * kTileSteps;
  const auto x_r = rsrc(x, (uint32_t)((int64_t)tokens * row_bytes));
  const int tiles = waves / runs;
  const auto xt_r = rsrc(xt, (uint32_t)((int64_t)tiles * steps * 1024));
  const int lane = threadIdx.x & 63;
  const int t = tt * kTokTile + (lane & 15);
  const int k0 = 64 * s0 + 16 * (lane >> 4);
  u32x4 v[kTileSteps];
#pragma unroll
  for (int j = 0; j < kTileSteps; ++j) {
    const int k = k0 + 64 * j;
    const bool in_range = t < tokens && k < row_bytes;  // row_bytes % 16 == 0: whole chunks
    v[j] = __builtin_amdgcn_raw_buffer_load_b128(x_r, in_range ? t * row_bytes + k : (int)0x80000000, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < kTileSteps; ++j) {
    const int s = s0 + j;  // steps past the row are not stored (the copy holds `steps` steps per tile)
    const int off = s < steps ? ((s * tiles + tt) * 64 + lane) * 16 : (int)0x80000000;
    __builtin_amdgcn_raw_buffer_store_b128(v[j], xt_r, off, 0, kStreamStore);
  }
}

// One work item of the fused linear: generated blocks tile*KB .. tile*KB + KB - 1
// against token split `split` of token_split (every thread of the workgroup
// calls it; `lds` is the workgroup's kLinearLdsBytes).  `pitch` table rows
// (>= the tile's output rows; 16*NT when that fits in the LDS, else exact and
// the last row tile masked on read).  kEpi: the stores apply `ep` (a separate
// instantiation, so the plain kernels carry none of its code or registers).
// kRowTiles (KB = 2): the tile is rows tile*rows_per_tile .. + rows_per_tile - 1
// instead, whole rows that lie in the two generated blocks starting at the
// block of its first position (linear_rows_per_tile), so no row straddles two
// tiles: the generated positions outside the tile are dropped, every row is
// stored directly, and no partial dot products or combine are needed.
// KB = 3 (row tiles, linear_three_block_rows): three whole blocks hold a whole
// number of rows (in_features 3072: 32 rows, 1.5 times the rows per loaded x
// element of a two-block tile) but their table does not fit in the LDS: the
// first linear_lds_steps k steps are read from the LDS table, the rest from
// this workgroup's overflow in `partial`, written in MFMA B-operand order
// (per k step and row tile, 64 lanes x 16 bytes) and read with the x stream.
template <int L, int NT, bool kTiled, int KB, bool kEpi, bool kRowTiles = false, int KG = kGroup, int KD = kDepth>
__device__ __forceinline__ void linear_item(const __bf16* __restrict__ x, const __bf16* __restrict__ latent,
                                            __bf16* __restrict__ out, float* __restrict__ partial, int tokens,
                                            int in_f, int out_f, int n, uint32_t seed32, float scale,
                                            int token_split, int64_t nblocks, int pitch, int split, int64_t tile,
                                            const LinearEpi& ep, unsigned char* lds, int rows_per_tile = 0) {
  static_assert(!kRowTiles || KB == 2 || KB == 3, "row tiles span two or three generated blocks");
  static_assert(KB != 3 || (kRowTiles && kTiled), "three-block tiles are row tiles over the tiled x");
  const int64_t size = (int64_t)in_f * out_f;
  const int64_t tile_len = kRowTiles ? (int64_t)rows_per_tile * in_f : (int64_t)KB * kB;
  const int64_t g0 = tile * tile_len;                             // first flat position
  const int64_t g1 = (g0 + tile_len < size) ? g0 + tile_len : size;  // one past the last
  const int64_t b_first = g0 >> kLog;                             // first generated block
  const int o_first = (int)(g0 / in_f);
  const int o_last = (int)((g1 - 1) / in_f);
  const bool first_partial = !kRowTiles && (g0 % in_f) != 0;
  const bool last_partial = !kRowTiles && (g1 % in_f) != 0;
  // k steps, padded to whole prefetch rounds: the padding reads zeros (table
  // rows past the row length are zero, x offsets past it are out of range)
  const int nsteps = linear_steps(in_f);
  const int kchunks = 4 * nsteps;  // 8-element k chunks per table row
  // three-block tiles: the k steps read from the LDS table, and this work
  // item's overflow (its own region of `partial`: work item split * tiles + tile)
  const int lds_steps = KB == 3 ? linear_lds_steps(nsteps, pitch) : nsteps;
  const uint32_t ovf_bytes = KB == 3 ? (uint32_t)(nsteps - lds_steps) * NT * 1024u : 0u;
  const int64_t item = KB == 3 ? split * (int64_t)((out_f + rows_per_tile - 1) / rows_per_tile) + tile : 0;
  unsigned char* item_ws = reinterpret_cast<unsigned char*>(partial) + item * (ovf_bytes + (KB == 3 ? kStageBytes : 0));
  const auto ovf_r = rsrc(item_ws, ovf_bytes);
  const auto stage_r = rsrc(item_ws + ovf_bytes, KB == 3 ? (uint32_t)kStageBytes : 0u);

  // 1. generate the tile's blocks (signed bf16; the first kept in registers
  //    while the next one's chain uses the LDS) and scatter them into LDS as a
  //    k-major table of 16-byte chunks: table[table_slot(kc, r, pitch)]
  //    holds W[o_first + r][8*kc .. 8*kc+7]; entries of the tile's rows outside
  //    [g0, g1) read 0.
  u32x4* table = reinterpret_cast<u32x4*>(lds);
  {
    const int nrows = o_last - o_first + 1;
    const int row_chunks = in_f >> 3;                   // chunks holding data in a row
    const int c_first = (int)(g0 - (int64_t)o_first * in_f) >> 3;  // first chunk of row 0 in the tile
    const int c_last = (int)(g1 - (int64_t)o_last * in_f) >> 3;    // chunks of the last row in the tile
    // block position p of generated block kb -> offset rel = off + kb * kB + p from the
    // start of row o_first (block tiles: off = the tile's start in that row; row tiles:
    // the first block's start, at or before g0), row r = rel / in_f (|rel| < in_f +
    // KB * kB: float quotient, corrected by one); kept where g0 <= flat < g1
    const int base_rel = c_first << 3;
    const int off = kRowTiles ? (int)((b_first << kLog) - g0) : base_rel;
    const int rel_lo = base_rel, rel_hi = (int)(g1 - (int64_t)o_first * in_f);
    const float inv_in = 1.0f / (float)in_f;
    u32x4 v[KB][8];
    const bool two = kRowTiles ? g1 > ((b_first + 1) << kLog) : (KB == 2 && tile * KB + 1 < nblocks);
    if constexpr (KB == 3) {
      // The first block alone, then the other two together (`run_chain2`;
      // each chain reuses the LDS once every wave has read the previous one's
      // last exchange).  The first block's chunks wait in this work item's
      // staging area (8 coalesced 16-byte stores per thread) while the pair
      // runs, and come back with all 8 loads in flight at once: kept in
      // registers through the pair chain they would be spilled, and the
      // compiler reloads spilled registers one memory round trip at a time.
      // The last tile of a matrix may generate blocks past its end, whose
      // positions are dropped.
      {
        const Ctx c0 = make_ctx(seed32, b_first);
        u32x4 src[kTiles][2];
        load_latent(c0, latent, n, src);
        f32x16 acc[kTiles];
        uint32_t nw[4];
        run_chain<L>(acc, c0, lds, src, [](int i) { return i; }, nw);
        out_chunks<L>(acc, nw, c0, v[0]);
#pragma unroll
        for (int k = 0; k < 8; ++k)
          __builtin_amdgcn_raw_buffer_store_b128(v[0][k], stage_r, (k * kThreads + threadIdx.x) * 16, 0, 0);
      }
      __syncthreads();
      {
        const Ctx c[2] = {make_ctx(seed32, b_first + 1), make_ctx(seed32, b_first + 2)};
        u32x4 src[kTiles][2];
        load_latent(c[0], latent, n, src);
        f32x16 acc[2][kTiles];
        uint32_t nw[2][4];
        run_chain2<L>(acc, c, lds, src, [](int i) { return i; }, nw);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) out_chunks<L>(acc[kb], nw[kb], c[kb], v[kb + 1]);
      }
#pragma unroll
      for (int k = 0; k < 8; ++k)
        v[0][k] = __builtin_amdgcn_raw_buffer_load_b128(stage_r, (k * kThreads + threadIdx.x) * 16, 0, 0);
    } else if (KB == 2 && two) {  // both blocks at once (uniform across the workgroup)
      const Ctx c[2] = {make_ctx(seed32, b_first), make_ctx(seed32, b_first + 1)};
      u32x4 src[kTiles][2];
      load_latent(c[0], latent, n, src);
      f32x16 acc[2][kTiles];
      uint32_t nw[2][4];
      run_chain2<L>(acc, c, lds, src, [](int i) { return i; }, nw);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) out_chunks<L>(acc[kb], nw[kb], c[kb], v[kb]);
    } else {  // one block (KB = 1, the last tile of an odd block count, or a row tile inside one block)
      const Ctx c = make_ctx(seed32, b_first);
      u32x4 src[kTiles][2];
      load_latent(c, latent, n, src);
      f32x16 acc[kTiles];
      uint32_t nw[4];
      run_chain<L>(acc, c, lds, src, [](int i) { return i; }, nw);
      out_chunks<L>(acc, nw, c, v[0]);
    }
    __syncthreads();  // every wave has read its last exchange
    // Zero exactly the entries of the tile's rows that the scatter leaves out
    // (disjoint from it, so no barrier in between): chunks before the tile's
    // start in row 0 and from its end in the last row, and k padding.  Rows
    // past the last one stay as they are (their output columns are not stored).
    // Three-block tiles are whole rows with no k padding (in_features % 128 == 0).
    if constexpr (KB != 3) {
      const int n_edge = 2 * kchunks;  // rows 0 and nrows - 1, every kc
      for (int i = threadIdx.x; i < n_edge; i += kThreads) {
        const int e = i >= kchunks;
        const int kc = i - e * kchunks;
        const int r = e ? nrows - 1 : 0;
        const int lo = r == 0 ? c_first : 0;
        const int hi = r == nrows - 1 ? c_last : row_chunks;
        if (kc < lo || kc >= hi) table[table_slot(kc, r, pitch)] = u32x4{0u, 0u, 0u, 0u};
      }
      // k padding of the inner rows (only when the row length is not a whole number of prefetch rounds)
      const int n_kpad = (kchunks - row_chunks) * (nrows > 2 ? nrows - 2 : 0);
      for (int i = threadIdx.x; i < n_kpad; i += kThreads) {
        const int q = kchunks - row_chunks;
        const int r = 1 + i / q, kc = row_chunks + (i - (i / q) * q);
        table[table_slot(kc, r, pitch)] = u32x4{0u, 0u, 0u, 0u};
      }
    }
    const Ctx c = make_ctx(seed32, b_first);  // chunk positions do not depend on the block
    if (KB == 3 || in_f % 32 == 0) {
      // A lane's chunk k = i + G g sits at block position out_chunk_pos(0) + 8 i
      // + GS g: G consecutive chunks per group.  With in_features % 32 == 0 the
      // tile's start in its first row, its end, the block starts and so every
      // group start are multiples of 8 G positions from a row start (three-block
      // tiles: in_features % 128 == 0), so a group lies in one row, one k step
      // and one side of the tile's edges (kc of its first chunk a multiple of G,
      // and of 4 when G = 4): one row and one LDS-or-overflow choice per group,
      // rows and columns advanced by adding GS's and the block length's quotient
      // and remainder by in_features.
      constexpr int G = L % 2 == 1 ? 2 : 4, GS = L % 2 == 1 ? 8192 : 2048, NG = 8 / G;
      const int q_g = GS / in_f, m_g = GS - q_g * in_f;
      const int q_b = kB / in_f, m_b = kB - q_b * in_f;
      const int rel0 = off + out_chunk_pos<L>(c, 0);
      int r0 = (int)((float)rel0 * inv_in);
      r0 -= r0 * in_f > rel0;
      r0 += (r0 + 1) * in_f <= rel0;
      const int col0 = rel0 - r0 * in_f;
#pragma unroll
      for (int kbi = 0; kbi < KB; ++kbi) {
        // three-block tiles scatter the staged first block last, so its reloads
        // arrive while the other two blocks' chunks go out
        const int kb = KB == 3 ? (kbi + 1) % 3 : kbi;
        if (KB == 2 && kRowTiles && kb > 0 && !two) break;  // uniform: no second block
        int r = r0 + kb * q_b, col = col0 + kb * m_b;
        if (kb == 2 && col >= 2 * in_f) { col -= in_f; ++r; }
        if (col >= in_f) { col -= in_f; ++r; }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          if (g > 0) {
            r += q_g;
            col += m_g;
            if (col >= in_f) { col -= in_f; ++r; }
          }
          const int rel = rel0 + kb * kB + g * GS;
          if (rel >= rel_lo && rel < rel_hi) {
            const int kc = col >> 3;
            if (KB != 3 || kc < 4 * lds_steps) {
              // odd chunks of a group: table_row's permuted row, one k chunk on
              const int s0 = kc * pitch + r + (kc >> 2), s1 = s0 + pitch + table_row(1, r, pitch) - r;
#pragma unroll
              for (int i = 0; i < G; ++i) table[(i & 1 ? s1 : s0) + (i >> 1) * 2 * pitch] = v[kb][i + G * g];
            } else {  // overflow: k step kc / 4, row tile r / 16, lane (r % 16) + 16 (kc % 4)
              const int e = (((kc >> 2) - lds_steps) * NT + (r >> 4)) * 64 + (r & 15) + 16 * (kc & 3);
#pragma unroll
              for (int i = 0; i < G; ++i)
                __builtin_amdgcn_raw_buffer_store_b128(v[kb][i + G * g], ovf_r, (e + 16 * i) * 16, 0, 0);
            }
          }
        }
      }
    } else if constexpr (KB != 3) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (KB == 2 && kRowTiles && kb > 0 && !two) break;  // uniform: no second block
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int rel = off + kb * kB + out_chunk_pos<L>(c, k);
          int r = (int)((float)rel * inv_in);
          r -= r * in_f > rel;
          r += (r + 1) * in_f <= rel;
          const int kc = (rel - r * in_f) >> 3;
          // chunks of 8 positions lie wholly inside or outside [g0, g1) (all multiples of 8)
          if (rel >= rel_lo && rel < rel_hi) table[table_slot(kc, r, pitch)] = v[kb][k];
        }
      }
    }
  }
  __syncthreads();

  // 2. this workgroup's token tiles
  const int ntiles_tok = (tokens + kTokTile - 1) / kTokTile;
  const int per_split = (ntiles_tok + token_split - 1) / token_split;
  const int tt0 = split * per_split;
  const int tt1 = (tt0 + per_split < ntiles_tok) ? tt0 + per_split : ntiles_tok;
  // the wave index as a scalar: the token tiles, and so the buffer resources of
  // the epilogue's stores, are then known to be uniform across the wave
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, kq = lane >> 4;  // A/B: row/col l16, k = 8*kq + j
  // x: the tiled copy (kTiled) or the row-major input; offsets past the end read 0
  const int xsteps = (in_f + kKStep - 1) / kKStep;
  const int ntiles_all = (tokens + kTokTile - 1) / kTokTile;
  const auto x_r = rsrc(x, kTiled ? (uint32_t)((int64_t)ntiles_all * xsteps * 1024)
                                  : (uint32_t)((int64_t)tokens * in_f * 2));
  float* part_first = partial + (tile * 2 + 0) * (int64_t)tokens;
  float* part_last = partial + (tile * 2 + 1) * (int64_t)tokens;
  // This lane's row of row tile nt at step s: brow + s * (4 * pitch + 1) + 16 nt
  // + dnt[nt].  Rows inside the table go through table_slot; rows past it (an
  // exact pitch, or a grouped job with fewer row tiles than the launch) read
  // their tile's first row, or row 0 when the whole tile lies past the table:
  // the same address as another lane of the LDS cycle, so no bank conflict.
  // Rows past the tile's last row are read as they are: W row o only feeds
  // output column o of the MFMA, and the epilogue stores no column past o_last,
  // so no load waits on a mask before the next step's MFMAs.
  const int slot_l16 = table_slot(kq, l16, pitch);
  const u32x4* brow = table + slot_l16;
  int dnt[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int r = 16 * nt + l16;
    const int rr = r < pitch ? r : (16 * nt < pitch ? 16 * nt : 0);
    dnt[nt] = table_slot(kq, rr, pitch) - slot_l16 - 16 * nt;
  }
  // row tiles: the table is 16 NT whole rows, so every dnt is 0
  auto brd = [&](const u32x4* b, int nt) -> u32x4 { return kRowTiles ? b[16 * nt] : b[16 * nt + dnt[nt]]; };
  constexpr uint32_t kOff = 0x80000000u;  // voffset that reads 0
  // epilogue: which terms, the row-sum coefficient (one scalar load), the bias
  const bool has_xs = kEpi && ep.xsum != nullptr, has_base = kEpi && ep.base != nullptr,
             has_bias = kEpi && ep.bias != nullptr;
  const float cx = has_xs ? ep.cscale * *ep.coef : 0.f;
  const auto bias_r = rsrc(has_bias ? ep.bias : (const void*)out, has_bias ? (uint32_t)(out_f * 2) : 0u);

  // A pass takes G consecutive token tiles (16 G tokens) of this wave: per k
  // step it reads the NT W tiles once from LDS and issues G * NT MFMAs; x is
  // prefetched D steps ahead into a register ring.  A single-tile pass (G = 1)
  // holds kDepthSingle steps in flight: it has few MFMAs per load, and at
  // decode it is the whole contraction of a workgroup, so its loop would
  // otherwise wait out one load latency per D steps.  Steps past nsteps (D need
  // not divide it) load x as 0 and reuse the last step's W, adding 0.  The
  // loop body has no branches, so the compiler can count the loads in flight.
  // Tiles from `tend` on are masked.
  auto pass = [&](auto g_const, int tg, int tend) {
    constexpr int G = decltype(g_const)::value;
    constexpr int D = (G == 1 && KB != 3) ? kDepthSingle : KD;
    uint32_t xo[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int tt = tg + g, t = tt * kTokTile + l16;
      if constexpr (kTiled)
        xo[g] = tt < tend ? (uint32_t)((tt * 64 + lane) * 16) : kOff;
      else
        xo[g] = (tt < tend && t < tokens) ? (uint32_t)((t * in_f + 8 * kq) * 2) : kOff;
    }
    // steps past the row (row-major: the lanes whose 8 k-values lie past it,
    // all or none as in % 8 == 0) read 0
    auto xload = [&](int g, int step) -> u32x4 {
      if constexpr (kTiled) {
        const uint32_t off = step < xsteps ? xo[g] : kOff;
        return __builtin_amdgcn_raw_buffer_load_b128(x_r, (int)off, step * ntiles_all * 1024, 0);
      } else {
        const uint32_t off = (step * kKStep + 8 * kq < in_f) ? xo[g] : kOff;
        return __builtin_amdgcn_raw_buffer_load_b128(x_r, (int)off, step * kKStep * 2, 0);
      }
    };
    f32x4v acc[G][NT];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[g][nt] = f32x4v{0.f, 0.f, 0.f, 0.f};
    // three-block tiles: the W tiles of the overflow steps (lds_steps on), D
    // steps ahead like x; the first D are loaded first, so they have arrived
    // by the time the loop waits for its x
    auto wload = [&](int nt, int step) -> u32x4 {
      const uint32_t off = step < nsteps ? (uint32_t)(lane * 16) : kOff;
      return __builtin_amdgcn_raw_buffer_load_b128(ovf_r, (int)off, ((step - lds_steps) * NT + nt) * 1024, 0);
    };
    u32x4 wring[KB == 3 ? D : 1][NT];
    if constexpr (KB == 3) {
#pragma unroll
      for (int d = 0; d < D; ++d)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) wring[d][nt] = wload(nt, lds_steps + d);
    }
    // Issue the first KD steps' loads in slot order, the order the loop
    // refills them in: the wait counts the compiler derives at the loop
    // head then let slot d's data arrive behind the later slots' requests.
    u32x4 ring[D][G];
#pragma unroll
    for (int d = 0; d < D; ++d) {
#pragma unroll
      for (int g = 0; g < G; ++g) ring[d][g] = xload(g, d);
      __builtin_amdgcn_sched_barrier(0);
    }
    // W tiles of step s are read one step ahead (bt holds step s, bn step s + 1),
    // so no MFMA waits on a just-issued LDS read; the last step re-reads itself.
    const u32x4* bs = brow;
    u32x4 bt[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) bt[nt] = brd(bs, nt);
    for (int s0 = 0; s0 < lds_steps; s0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int sn = (s0 + d + 1 < lds_steps) ? s0 + d + 1 : lds_steps - 1;
        const u32x4* bsn = brow + sn * (4 * pitch + 1);
        u32x4 bn[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) bn[nt] = brd(bsn, nt);
        bs = bsn;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) acc[g][nt] = mfma16(ring[d][g], bt[nt], acc[g][nt]);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) bt[nt] = bn[nt];
        // Refill slot d only after its last use, so the load writes the
        // slot's own registers: a load issued earlier would need a second
        // register set and a copy (with a wait on the fresh load) at the
        // loop back-edge, which serialises the whole prefetch.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < G; ++g) ring[d][g] = xload(g, s0 + d + D);
      }
    }
    if constexpr (KB == 3) {
      // the overflow steps: W from the ring, refilled with x (lds_steps and
      // nsteps are whole prefetch rounds; loads past nsteps read 0)
      for (int s0 = lds_steps; s0 < nsteps; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[g][nt] = mfma16(ring[d][g], wring[d][nt], acc[g][nt]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int g = 0; g < G; ++g) ring[d][g] = xload(g, s0 + d + D);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) wring[d][nt] = wload(nt, s0 + d + D);
        }
      }
    }
    // D[m = 4*kq + r][n = l16]: token 16 tt + 4 kq + r, row o_first + 16 nt + l16.
    // Branch-free stores: each token tile gets buffer resources over its own rows
    // of out and of the partials (tokens past the end fall outside them), and an
    // element that does not belong in a destination gets the offset that drops it.
    // The epilogue's inputs are read the same way (out-of-range reads give 0).
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int tt = tg + g;
      if (tt >= tend) continue;  // uniform across the wave
      const int t0 = tt * kTokTile;
      const int nt_tok = tokens - t0 < kTokTile ? tokens - t0 : kTokTile;
      const auto o_r = rsrc(out + (int64_t)t0 * out_f, (uint32_t)(nt_tok * out_f * 2));
      const auto pf_r = rsrc(part_first + t0, (uint32_t)(nt_tok * 4));
      const auto pl_r = rsrc(part_last + t0, (uint32_t)(nt_tok * 4));
      const auto xs_r = rsrc(has_xs ? (const void*)(ep.xsum + t0) : (const void*)out, has_xs ? (uint32_t)(nt_tok * 4) : 0u);
      const auto b_r = rsrc(has_base ? (const __bf16*)ep.base + (int64_t)t0 * out_f : out,
                            has_base ? (uint32_t)(nt_tok * out_f * 2) : 0u);
      auto out_off = [&](int nt, int r) {  // byte offset of (token 4 kq + r, row tile nt) in out, or kOff
        const int o = o_first + 16 * nt + l16;
        const bool is_out = o <= o_last && !(first_partial && o == o_first) && !(last_partial && o == o_last);
        return is_out ? ((4 * kq + r) * out_f + o) * 2 : (int)kOff;
      };
      // The epilogue's inputs of the whole token tile are loaded before its
      // first store: a load issued after a store that may alias it waits for
      // that store, which would serialize one memory round trip per element.
      // No load sits behind a branch on its term (a branched load is waited
      // for on its own): an absent term's buffer is empty and reads 0.  With
      // five or six row tiles the base values all in flight would spill, so
      // there base and bias keep their branches.
      float xs[4] = {0.f, 0.f, 0.f, 0.f}, base_v[NT][4], bias_v[NT];
      if constexpr (kEpi) {
        constexpr bool kFlat = NT <= 4;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          xs[r] = cx * __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xs_r, (4 * kq + r) * 4, 0, 0));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          bias_v[nt] = (kFlat || has_bias) ? bf16_at(bias_r, (o_first + 16 * nt + l16) * 2) : 0.f;
#pragma unroll
          for (int r = 0; r < 4; ++r) base_v[nt][r] = (kFlat || has_base) ? bf16_at(b_r, out_off(nt, r)) : 0.f;
        }
      }
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int o = o_first + 16 * nt + l16;
        const bool is_first = first_partial && o == o_first;
        const bool is_last = last_partial && o == o_last;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = scale * acc[g][nt][r];
          if constexpr (kEpi) v = linear_epilogue(v, has_xs, xs[r], has_base, base_v[nt][r], has_bias, bias_v[nt]);
          const uint16_t b = __builtin_bit_cast(uint16_t, (__bf16)v);
          __builtin_amdgcn_raw_buffer_store_b16(b, o_r, out_off(nt, r), 0, 0);
        }
        // partial rows: the first row of the tile (nt 0, l16 0) and its last row
        if (!kRowTiles && (nt == 0 || 16 * (nt + 1) > o_last - o_first)) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = 4 * kq + r;
            const uint32_t bits = __float_as_uint(acc[g][nt][r]);
            __builtin_amdgcn_raw_buffer_store_b32(bits, pf_r, is_first ? m * 4 : (int)kOff, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b32(bits, pl_r, is_last ? m * 4 : (int)kOff, 0, 0);
          }
        }
      }
    }
  };

  // Whole rounds in which every wave takes KG tiles, then the remainder.  With
  // three or more row tiles, or fewer remaining tiles than waves (decode), the
  // remainder is split evenly over the waves in single-tile passes (a round with
  // only some waves busy would leave the CU's other SIMDs idle for a whole
  // KG-tile pass); otherwise, with one or two row tiles, a single-tile pass has
  // too few MFMAs per load, and the remainder runs as KG-tile passes.
  const int full = (tt1 - tt0) / (KG * kWaves);
  for (int r = 0; r < full; ++r) pass(std::integral_constant<int, KG>{}, tt0 + (r * kWaves + wave) * KG, tt1);
  const int rest0 = tt0 + full * KG * kWaves;
  if (NT >= 3 || tt1 - rest0 <= kWaves) {
    const int per = (tt1 - rest0 + kWaves - 1) / kWaves;
    for (int i = 0; i < per; ++i) {
      const int tt = rest0 + wave * per + i;
      if (tt < tt1) pass(std::integral_constant<int, 1>{}, tt, tt1);  // uniform across the wave
    }
  } else {
    for (int tg = rest0 + KG * wave; tg < tt1; tg += KG * kWaves) pass(std::integral_constant<int, KG>{}, tg, tt1);
  }
}
template <int L, int NT, bool kTiled, int KB, bool kEpi, bool kRowTiles = false, int KG = kGroup, int KD = kDepth>
__global__ __launch_bounds__(kThreads) void bfht_linear_mfma15(const __bf16* __restrict__ x,
                                                               const __bf16* __restrict__ latent,
                                                               __bf16* __restrict__ out,
                                                               float* __restrict__ partial, int tokens,
                                                               int in_f, int out_f, int n, uint32_t seed32,
                                                               float scale, int token_split, int64_t nblocks,
                                                               int pitch, LinearEpi ep, int rows_per_tile) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLinearLdsBytes];
  // XCD-aware work order: workgroup i runs on XCD i % 8, and work item
  // p = split * ntiles + tile (split-major) goes to XCD p / per_xcd, so each
  // XCD's L2 holds the x rows of one or two token splits instead of all of x.
  const int64_t ntiles = kRowTiles ? (out_f + rows_per_tile - 1) / rows_per_tile : (nblocks + KB - 1) / KB;
  const int64_t nwork = ntiles * token_split;
  const int64_t per_xcd = (nwork + kXcds - 1) / kXcds;
  const int64_t p = (int64_t)(blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
  if (p >= nwork) return;  // uniform: the grid is rounded up to whole XCD rows
  const int split = (int)(p / ntiles);
  const int64_t tile = p - (int64_t)split * ntiles;
  linear_item<L, NT, kTiled, KB, kEpi, kRowTiles, KG, KD>(x, latent, out, partial, tokens, in_f, out_f, n, seed32,
                                                          scale, token_split, nblocks, pitch, split, tile, ep, lds,
                                                          rows_per_tile);
}

// Output (t, o) of a straddling row from its two partial dot products, with the epilogue.
__device__ __forceinline__ float combine_value(float p_last, float p_first, float scale, const LinearEpi& ep, int t,
                                               int o, int out_f) {
  const bool has_xs = ep.xsum != nullptr, has_base = ep.base != nullptr, has_bias = ep.bias != nullptr;
  const float xs = has_xs ? ep.cscale * *ep.coef * ep.xsum[t] : 0.f;
  const float base_v = has_base ? (float)((const __bf16*)ep.base)[(int64_t)t * out_f + o] : 0.f;
  const float bias_o = has_bias ? (float)((const __bf16*)ep.bias)[o] : 0.f;
  return linear_epilogue(scale * (p_last + p_first), has_xs, xs, has_base, base_v, has_bias, bias_o);
}

// Rows straddling tiles b-1 and b: out[t][o] = scale * (last(b-1)[t] + first(b)[t]) + epilogue.
__global__ __launch_bounds__(256) void bfht_linear_combine(const float* __restrict__ partial,
                                                           __bf16* __restrict__ out, int tokens, int in_f,
                                                           int out_f, int64_t ntiles, int64_t tile_len,
                                                           float scale, LinearEpi ep) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int64_t b = (int64_t)blockIdx.y + 1;
  if (t >= tokens || b >= ntiles) return;
  const int64_t g0 = b * tile_len;
  if (g0 % in_f == 0) return;
  const int o = (int)(g0 / in_f);
  const float v = combine_value(partial[((b - 1) * 2 + 1) * (int64_t)tokens + t], partial[(b * 2) * (int64_t)tokens + t],
                                scale, ep, t, o, out_f);
  store_bf16_through(out + (int64_t)t * out_f + o, v);
}

// Several matrices in one launch (the decode case: each matrix has a few dozen
// generated blocks, far fewer than the 256 CUs): workgroup i serves job j with
// prefix[j] <= i < prefix[j + 1], work item i - prefix[j] = split * nblocks +
// block, as the single-matrix kernel's non-tiled, one-block-per-workgroup path
// (kBias: some job has a bias, applied as the single call's epilogue).
template <int L, int NT, bool kBias>
__global__ __launch_bounds__(kThreads) void bfht_linear_mfma15_grouped(const LinearGroupTable g) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLinearLdsBytes];
  const int j = group_job(g, (int)blockIdx.x);
  const LinearGroupJob& jb = g.job[j];
  const int64_t p = (int64_t)blockIdx.x - g.prefix[j];
  const int split = (int)(p / jb.nblocks);
  const int64_t tile = p - (int64_t)split * jb.nblocks;
  const LinearEpi ep{jb.bias, nullptr, nullptr, nullptr, 0.f};
  linear_item<L, NT, false, 1, kBias>(jb.x, jb.latent, jb.out, g.partial + jb.partial_off, jb.tokens, jb.in_f, jb.out_f,
                               jb.n, jb.seed32, jb.scale, jb.token_split, jb.nblocks, jb.pitch, split, tile, ep, lds);
}

// The straddling-row sums of every job of a grouped launch: workgroup i serves
// job j with cprefix[j] <= i < cprefix[j + 1], one thread per (block boundary,
// token) pair of the job, tokens fastest (a decode job's boundaries share one
// workgroup), with the arithmetic of bfht_linear_combine.
__global__ __launch_bounds__(256) void bfht_linear_combine_grouped(const LinearGroupTable g) {
  int j = 0;
  while (j + 1 < g.count && (int)blockIdx.x >= g.cprefix[j + 1]) ++j;
  const LinearGroupJob& jb = g.job[j];
  const int64_t i = (int64_t)((int)blockIdx.x - g.cprefix[j]) * 256 + threadIdx.x;
  if (i >= (int64_t)(jb.nblocks - 1) * jb.tokens) return;
  const int64_t b = i / jb.tokens + 1;
  const int t = (int)(i - (b - 1) * jb.tokens);
  const int64_t g0 = b * kB;
  if (g0 % jb.in_f == 0) return;
  const int o = (int)(g0 / jb.in_f);
  const float* partial = g.partial + jb.partial_off;
  const LinearEpi ep{jb.bias, nullptr, nullptr, nullptr, 0.f};
  const float v = combine_value(partial[((b - 1) * 2 + 1) * (int64_t)jb.tokens + t], partial[(b * 2) * (int64_t)jb.tokens + t],
                                jb.scale, ep, t, o, jb.out_f);
  store_bf16_through(jb.out + (int64_t)t * jb.out_f + o, v);
}

template <int L, bool kTiled, int KB, bool kEpi, bool kRowTiles = false>
hipError_t launch_linear_kb(const LinearArgs& a, const __bf16* x, float* partial, hipStream_t s) {
  const int R = a.rows_per_tile;
  const int nt = kRowTiles ? (R + 15) / 16 : (int)linear_row_tiles(a.in_features, KB);
  const int64_t ntiles = kRowTiles ? (a.out_features + R - 1) / R : (a.nblocks_w + KB - 1) / KB;
  const int pitch = kRowTiles ? 16 * nt : linear_pitch(a.in_features, KB);
  const int64_t per_xcd = (ntiles * a.token_splits + kXcds - 1) / kXcds;
  const dim3 grid((unsigned)(per_xcd * kXcds)), block(mfma15::kThreads);
  auto* lat = (const __bf16*)a.latent;
  auto* o = (__bf16*)a.out;
#define LWL_LIN(NT)                                                                                               \
  hipLaunchKernelGGL((bfht_linear_mfma15<L, NT, kTiled, KB, kEpi, kRowTiles>), \
                     grid, block, 0, s, x, lat, o, partial,                                                      \
                     (int)a.tokens, (int)a.in_features, (int)a.out_features, (int)a.n, a.seed32, a.weight_scale, \
                     a.token_splits, a.nblocks_w, pitch, a.epi, R)
  switch (nt) {
    case 1: LWL_LIN(1); break;
    case 2: LWL_LIN(2); break;
    case 3: if constexpr (KB != 3) LWL_LIN(3); else return hipErrorInvalidValue; break;
    case 4: if constexpr (KB != 3) LWL_LIN(4); else return hipErrorInvalidValue; break;
    case 5: if constexpr (KB == 2) LWL_LIN(5); else return hipErrorInvalidValue; break;
    case 6: if constexpr (KB == 2) LWL_LIN(6); else return hipErrorInvalidValue; break;
    default: return hipErrorInvalidValue;
  }
#undef LWL_LIN
  hipError_t e = hipGetLastError();
  // no row straddles two tiles: row tiles, or block tiles whose length is a whole number of rows
  if (e != hipSuccess || ntiles < 2 || kRowTiles || ((int64_t)KB * mfma15::kB) % a.in_features == 0) return e;
  hipLaunchKernelGGL(bfht_linear_combine, dim3((unsigned)((a.tokens + 255) / 256), (unsigned)(ntiles - 1)),
                     dim3(256), 0, s, (const float*)partial, o, (int)a.tokens, (int)a.in_features,
                     (int)a.out_features, ntiles, (int64_t)KB * mfma15::kB, a.weight_scale, a.epi);
  return hipGetLastError();
}

template <int L, bool kTiled, bool kEpi>
hipError_t launch_linear_e(const LinearArgs& a, const __bf16* x, float* partial, hipStream_t s) {
  if constexpr (kTiled) {
    if (a.blocks_per_wg == 3) return launch_linear_kb<L, true, 3, kEpi, true>(a, x, partial, s);
    if (a.blocks_per_wg == 2 && a.rows_per_tile > 0) return launch_linear_kb<L, true, 2, kEpi, true>(a, x, partial, s);
    if (a.blocks_per_wg == 2) return launch_linear_kb<L, true, 2, kEpi>(a, x, partial, s);
  }
  return launch_linear_kb<L, kTiled, 1, kEpi>(a, x, partial, s);
}

template <int L, bool kTiled>
hipError_t launch_linear_L(const LinearArgs& a, const __bf16* x, float* partial, hipStream_t s) {
  if (a.epi.bias || a.epi.base || a.epi.xsum) return launch_linear_e<L, kTiled, true>(a, x, partial, s);
  return launch_linear_e<L, kTiled, false>(a, x, partial, s);
}

template <int L>
hipError_t launch_linear_L(const LinearArgs& a, hipStream_t s) {
  float* partial = (float*)a.work;
  if (!linear_tiled(a)) return launch_linear_L<L, false>(a, (const __bf16*)a.x, partial, s);
  auto* tiled = reinterpret_cast<u32x4*>((unsigned char*)a.work + partial_bytes(a));
  const hipError_t e = launch_tile_x(a.x, tiled, a.tokens, a.in_features * 2, s);
  if (e != hipSuccess) return e;
  return launch_linear_L<L, true>(a, (const __bf16*)tiled, partial, s);
}

template <int L, bool kBias>
hipError_t launch_grouped_b(const LinearGroupTable& g, int nt, hipStream_t s) {
  const dim3 grid((unsigned)g.prefix[g.count]), block(mfma15::kThreads);
  switch (nt) {
    case 1: hipLaunchKernelGGL((bfht_linear_mfma15_grouped<L, 1, kBias>), grid, block, 0, s, g); break;
    case 2: hipLaunchKernelGGL((bfht_linear_mfma15_grouped<L, 2, kBias>), grid, block, 0, s, g); break;
    case 3: hipLaunchKernelGGL((bfht_linear_mfma15_grouped<L, 3, kBias>), grid, block, 0, s, g); break;
    case 4: hipLaunchKernelGGL((bfht_linear_mfma15_grouped<L, 4, kBias>), grid, block, 0, s, g); break;
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}

template <int L>
hipError_t launch_grouped_nt(const LinearGroupTable& g, int nt, hipStream_t s) {
  bool bias = false;
  for (int i = 0; i < g.count; ++i) bias = bias || g.job[i].bias;
  const hipError_t e0 = bias ? launch_grouped_b<L, true>(g, nt, s) : launch_grouped_b<L, false>(g, nt, s);
  if (e0 != hipSuccess) return e0;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || g.cprefix[g.count] == 0) return e;
  hipLaunchKernelGGL(bfht_linear_combine_grouped, dim3((unsigned)g.cprefix[g.count]), dim3(256), 0, s, g);
  return hipGetLastError();
}

// Whether a job's k-major table can be read as `nt` row tiles: the contraction
// reads rows up to 16 nt - 1 of every k chunk (rows past the job's own are
// never stored), so the last chunk's reads reach 16 nt - pitch rows past its
// table; they must stay inside the workgroup's LDS.
bool table_reads_fit(const LinearArgs& a, int nt) {
  const int64_t pitch = linear_pitch(a.in_features, 1);
  const int64_t steps = linear_steps(a.in_features);
  const int64_t last = (4 * steps - 1) * pitch + (16 * nt - 1) + (4 * steps - 1) / 4;  // highest slot read
  return (last + 1) * 16 <= kLinearLdsBytes;
}

// One grouped launch (plus its combine) for jobs of one layer count, read as
// `nt` row tiles (the largest of the jobs').
hipError_t launch_group_chunk(const LinearArgs* const* jobs, int count, int nt, hipStream_t s) {
  LinearGroupTable g{};
  g.count = count;
  int64_t total = 0, min_tiles = INT64_MAX;
  for (int i = 0; i < count; ++i) {
    total += jobs[i]->nblocks_w;
    const int64_t tt = (jobs[i]->tokens + kTokTile - 1) / kTokTile;
    min_tiles = tt < min_tiles ? tt : min_tiles;
  }
  // one pass over every job's blocks fills the chip when there are >= 256 of
  // them; otherwise split the tokens, as the single-matrix launch does
  int64_t split = total >= 256 ? 1 : 256 / total;
  if (split > min_tiles) split = min_tiles;
  if (split < 1) split = 1;
  // partial rows: offsets from the lowest `work` (every job's lies in one
  // 256-byte-aligned workspace)
  g.partial = (float*)jobs[0]->work;
  for (int i = 1; i < count; ++i)
    if ((float*)jobs[i]->work < g.partial) g.partial = (float*)jobs[i]->work;
  int64_t wg = 0, cw = 0;
  for (int i = 0; i < count; ++i) {
    const LinearArgs& a = *jobs[i];
    LinearGroupJob& jb = g.job[i];
    jb.x = (const __bf16*)a.x;
    jb.latent = (const __bf16*)a.latent;
    jb.out = (__bf16*)a.out;
    jb.bias = (const __bf16*)a.epi.bias;
    jb.partial_off = (uint32_t)((float*)a.work - g.partial);
    jb.tokens = (int)a.tokens;
    jb.in_f = (int)a.in_features;
    jb.out_f = (int)a.out_features;
    jb.n = (int)a.n;
    jb.seed32 = a.seed32;
    jb.scale = a.weight_scale;
    jb.nblocks = (int)a.nblocks_w;
    jb.pitch = linear_pitch(a.in_features, 1);
    jb.token_split = (int)split;
    g.prefix[i] = (int)wg;
    g.cprefix[i] = (int)cw;
    wg += a.nblocks_w * split;
    cw += ((a.nblocks_w - 1) * a.tokens + 255) / 256;
  }
  g.prefix[count] = (int)wg;
  g.cprefix[count] = (int)cw;
  switch (jobs[0]->layers) {
    case 1: return launch_grouped_nt<1>(g, nt, s);
    case 2: return launch_grouped_nt<2>(g, nt, s);
    case 3: return launch_grouped_nt<3>(g, nt, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_tile_x(const void* x, void* xt, int64_t tokens, int64_t row_bytes, hipStream_t s) {
  const int64_t tiles = (tokens + kTokTile - 1) / kTokTile;
  const int steps = (int)((row_bytes + 63) / 64);
  const int runs = (steps + kTileSteps - 1) / kTileSteps;
  const int64_t waves = tiles * runs;
  hipLaunchKernelGGL(bfht_linear_tile_x, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s,
                     (const unsigned char*)x, (u32x4*)xt, (int)tokens, (int)row_bytes, steps, runs, (int)waves);
  return hipGetLastError();
}

bool linear_groupable(const LinearArgs& a) {
  return linear_applicable(a.dtype, a.log_block, a.in_features) && !linear_tiled(a);
}

hipError_t launch_linear_grouped(const LinearArgs* jobs, int64_t count, hipStream_t s) {
  // Buckets in job order: one per layer count, read as the largest row-tile
  // count among the pending jobs of that layer count (the extra row tiles of
  // smaller jobs cost MFMAs on rows that are never stored, little at the batch
  // sizes grouped here); jobs whose table cannot be read that wide wait for a
  // later bucket, and a bucket that would be empty falls back to the first
  // pending job's own row-tile count (which its single launch reads, so it
  // fits).  Every round launches at least one job.  At most kLinearGroupMax
  // jobs per launch.
  std::vector<bool> done((size_t)count, false);
  std::vector<const LinearArgs*> bucket;
  auto tiles = [&](int64_t k) { return (int)linear_row_tiles(jobs[k].in_features, 1); };
  for (;;) {
    int64_t i = 0;
    while (i < count && done[(size_t)i]) ++i;
    if (i == count) return hipSuccess;
    const int L = jobs[i].layers;
    int nt = 0;
    for (int64_t k = i; k < count; ++k)
      if (!done[(size_t)k] && jobs[k].layers == L) nt = std::max(nt, tiles(k));
    auto take = [&](int64_t k, int w) {
      return !done[(size_t)k] && jobs[k].layers == L && tiles(k) <= w && table_reads_fit(jobs[k], w);
    };
    bool any = false;
    for (int64_t k = i; k < count && !any; ++k) any = take(k, nt);
    if (!any) nt = tiles(i);
    bucket.clear();
    for (int64_t k = i; k < count; ++k) {
      if (!take(k, nt) && !(k == i && !any)) continue;
      done[(size_t)k] = true;
      bucket.push_back(&jobs[k]);
      if ((int)bucket.size() == kLinearGroupMax) {
        const hipError_t e = launch_group_chunk(bucket.data(), (int)bucket.size(), nt, s);
        if (e != hipSuccess) return e;
        bucket.clear();
      }
    }
    if (!bucket.empty()) {
      const hipError_t e = launch_group_chunk(bucket.data(), (int)bucket.size(), nt, s);
      if (e != hipSuccess) return e;
    }
  }
}

const bool kLinearKernelAvailable = true;

bool linear_applicable(int dtype, int log_block, int64_t in_features) {
  // bf16 matrix-core generator (B = 2^15); 16-byte rows of x and W (in % 8 == 0);
  // at most kMaxNT tiles of 16 rows per block; the k-major table fits in LDS.
  if (dtype != kBF16 || log_block != mfma15::kLog || in_features % 8 != 0 || in_features > mfma15::kB) return false;
  return in_features <= kLinearMaxIn && linear_row_tiles(in_features) <= kMaxNT && linear_pitch_fits(in_features, 1);
}

int linear_blocks_per_wg(const LinearArgs& a) {
  // Two blocks per workgroup for batches read from the tiled x copy when a block
  // holds at most 64 rows (the contraction is bound by streaming x, and two
  // blocks feed each x element twice the rows: at 768 -> 3072 the second chain
  // costs ~7 us and the contraction saves ~13), their rows fit the register
  // budget and their table the LDS.  Three when three blocks hold whole rows
  // (linear_three_block_rows) and the batch is large enough to pay the third chain.
  if (!linear_tiled(a) || a.nblocks_w < 2 || linear_rows(a.in_features, 1) > 64) return 1;
  if (a.nblocks_w >= 3 && a.tokens >= kThreeBlockMinTokens && linear_three_block_rows(a.in_features) > 0) return 3;
  if (linear_row_tiles(a.in_features, 2) > kMaxNT2) return 1;
  return linear_pitch_fits(a.in_features, 2) ? 2 : 1;
}

int linear_rows_per_tile(const LinearArgs& a) {
  // Tiles of R whole rows in place of two-block tiles whose ends split rows
  // (the straddling rows' partial sums and their combine launch, ~4.6 us at
  // 4096 tokens, go away): R a multiple of 16 of at least 48, with R * in at
  // least 1.5 blocks (about as many rows per loaded x element as two blocks
  // give), and every tile [j R in, (j + 1) R in) inside the two blocks from the
  // one holding its start, whose offset in that block is a multiple of
  // gcd(R in, 2^15) and at most 2^15 - gcd: R in + 2^15 - gcd <= 2^16.
  // GPT-2's rows of 768: R = 64 (1.5 blocks per tile).
  if (a.blocks_per_wg == 3) return linear_three_block_rows(a.in_features);
  if (a.blocks_per_wg != 2 || (2 * mfma15::kB) % a.in_features == 0) return 0;
  for (int R = 16 * kMaxNT2; R >= 48; R -= 16) {
    const int64_t len = (int64_t)R * a.in_features;
    int64_t g = len, b = mfma15::kB;  // gcd(len, 2^15)
    while (b) { const int64_t t = g % b; g = b; b = t; }
    if (2 * len >= 3 * mfma15::kB && len + mfma15::kB - g <= 2 * mfma15::kB &&
        linear_table_bytes(a.in_features, R) <= kLinearLdsBytes)
      return R;
  }
  return 0;
}

size_t linear_workspace_bytes(const LinearArgs& a) {
  return partial_bytes(a) + (linear_tiled(a) ? x_tiling(a).bytes() : 0);
}

int linear_token_splits(const LinearArgs& a) {
  // one workgroup per CU: split tokens so that block tiles x splits fills 256
  // CUs, never below one 16-token tile per split
  const int64_t tiles = (a.tokens + kTokTile - 1) / kTokTile;
  const int64_t wtiles = a.rows_per_tile > 0 ? (a.out_features + a.rows_per_tile - 1) / a.rows_per_tile
                                             : (a.nblocks_w + a.blocks_per_wg - 1) / a.blocks_per_wg;
  int64_t split = wtiles >= 256 ? 1 : 256 / wtiles;
  if (split > tiles) split = tiles;
  return (int)(split < 1 ? 1 : split);
}

hipError_t launch_linear(const LinearArgs& a, hipStream_t s) {
  switch (a.layers) {
    case 1: return launch_linear_L<1>(a, s);
    case 2: return launch_linear_L<2>(a, s);
    case 3: return launch_linear_L<3>(a, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace lwl
