// BlockFHT at block size 2^15 on the matrix cores (gfx950, bf16 operands,
// float32 accumulation).
//
// One workgroup (4 waves, one per SIMD) owns one 32768-element block; each
// lane holds 128 values as 8 MFMA accumulator tiles of 16 floats.  The
// normalized Hadamard transform of a layer is split over three 5-bit groups
// of the position index (H_32768 = H_32 (x) H_32 (x) H_32), each applied as a
// 32x32 Walsh matrix with v_mfma_f32_32x32x16_bf16:
//
//   stage a, b: data is the A operand (rows = lane, k = lane bit 5 + 4
//               register bits); the transformed group lands in the lane bits
//               and the old lane bits move into the registers;
//   stage c:    data is the B operand; its 5 bits include the two wave bits,
//               so it is preceded by one LDS exchange (64 KiB bf16) that swaps
//               two already-transformed bits out to the wave index.
//
// Slot -> position bit assignment (p0..p14; Lk = lane bit k, Rk = bit k of
// the accumulator register index r = 0..15, Tk = bit k of the tile index,
// Wk = wave bit k):
//
//   S0 (even layer start):  L0-4 = p5-9, L5 = p10, R = p0 p1 p2 p11, T = p3 p4 p12, W = p13 p14
//   S1 (odd layer start):   L0-4 = p5-9, L5 = p12, R = p3 p4 p13 p14, T = p0 p1 p2, W = p10 p11
//
// A layer started in S0 ends in S1 and vice versa, so every sign layer D_l
// meets the five bit-in-word position bits (p0..p4) in registers: the sign
// words (one 32-bit hash per 32 positions) are computed per lane, four per
// layer, and applied to packed bf16 pairs as XOR masks
// (word << (15 - b)) & 0x80008000 after a fixed permutation of the word's
// bits that matches the pair's position bit.
//
// The Walsh matrices use entries +-1/4, +-1/8, +-1/4 (exact in bf16); the
// remaining 2^(-L/2) of the L-layer normalization is folded into the last
// stage's entries (rounded to bf16, relative error <= 2^-9).
//
// Reference semantics: latent_weight_lab/block_fht.py:84-109 (forward) and
// csrc/block_fht_ext_cuda.cu:185-223 (backward: the same chain with the sign
// layers in reverse order).
#include "bfht_device.h"
#include "bfht_launch.h"

namespace lwl {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kLog = 15;
constexpr int kB = 1 << kLog;
constexpr int kThreads = 256;
constexpr uint32_t kPairSign = 0x80008000u;

__device__ __forceinline__ uint32_t pk(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Sign-word bit permutations: exchange bit-index bit 0 (resp. 3) with bit 4,
// so that the two positions of a packed pair sit 16 word bits apart.
__device__ __forceinline__ uint32_t swap_idx04(uint32_t x) {
  const uint32_t t = ((x >> 15) ^ x) & 0x0000aaaau;
  return x ^ t ^ (t << 15);
}
__device__ __forceinline__ uint32_t swap_idx34(uint32_t x) {
  const uint32_t t = ((x >> 8) ^ x) & 0x0000ff00u;
  return x ^ t ^ (t << 8);
}

// Walsh operand of this lane for a 32x32 stage: entry (c, j), k = 16c + 8*(lane>>5) + j,
// o = lane & 31, is scale * (-1)^popcount(remap(k) & o) where k bit i is o bit Mi.
// The same registers serve as B operand (o = column) and A operand (o = row).
template <int M0, int M1, int M2, int M3, int M4>
__device__ __forceinline__ void walsh_operand(int lane, float scale, u32x4 (&h)[2]) {
  const int o = lane & 31, hi = lane >> 5;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float e[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int k = 16 * c + 8 * hi + 2 * v + s;
        const int km = ((k & 1) << M0) | (((k >> 1) & 1) << M1) | (((k >> 2) & 1) << M2) |
                       (((k >> 3) & 1) << M3) | (((k >> 4) & 1) << M4);
        e[s] = (__popc(km & o) & 1) ? -scale : scale;
      }
      h[c][v] = pk(e[0], e[1]);
    }
  }
}

// Four sign words of one layer for this lane, inverted (set bit = flip) and
// permuted for the pair layout.  Even (S0): word index = base | c<<6 | t2<<7,
// slot = c + 2*t2.  Odd (S1): base | v1<<8 | c<<9, slot = v1 + 2*c.
template <bool kOdd>
__device__ __forceinline__ void layer_words(uint32_t bkey, int layer, uint32_t base, uint32_t (&nw)[4]) {
  const uint32_t lkey = layer_key(layer);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint32_t word = kOdd ? (base | ((uint32_t)(s & 1) << 8) | ((uint32_t)(s >> 1) << 9))
                               : (base | ((uint32_t)(s & 1) << 6) | ((uint32_t)(s >> 1) << 7));
    const uint32_t w = ~sign_word(bkey, lkey, word);
    nw[s] = kOdd ? swap_idx34(w) : swap_idx04(w);
  }
}

// XOR mask of stage-a operand VGPR v of tile t, instruction c.
template <bool kOdd>
__device__ __forceinline__ uint32_t operand_mask(const uint32_t (&nw)[4], int t, int c, int v) {
  if (kOdd) {
    const int b = t | ((v & 1) << 3);
    return (nw[(v >> 1) + 2 * c] << (15 - b)) & kPairSign;
  }
  const int b = ((t >> 1) & 1) | (v << 1) | ((t & 1) << 3);
  return (nw[c + 2 * (t >> 2)] << (15 - b)) & kPairSign;
}

__device__ __forceinline__ u32x4 pack8(const f32x16& a, int base) {
  u32x4 r;
  r[0] = pk(a[base + 0], a[base + 1]);
  r[1] = pk(a[base + 2], a[base + 3]);
  r[2] = pk(a[base + 4], a[base + 5]);
  r[3] = pk(a[base + 6], a[base + 7]);
  return r;
}

// Stage a of a layer whose input sits in acc: sign D_layer fused into the operands.
template <bool kOdd>
__device__ __forceinline__ void stage_rows_signed(f32x16 (&acc)[8], const u32x4 (&h)[2],
                                                  const uint32_t (&nw)[4]) {
  const f32x16 zero = {};
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    u32x4 a[2] = {pack8(acc[t], 0), pack8(acc[t], 8)};
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v) a[c][v] ^= operand_mask<kOdd>(nw, t, c, v);
    f32x16 d = mfma(a[0], h[0], zero);
    acc[t] = mfma(a[1], h[1], d);
  }
}

// Exchange chunk ids (16-byte chunks of 8 packed bf16, the values of the 8
// tiles at one accumulator register r): write side lane32 + (r&7)<<5 + l5<<8 +
// (r>>3)<<9 + wave<<10, read side lane32 + t<<5 + wave<<8 + l5<<10 + c<<11.
// Both are a per-lane base plus a compile-time constant.  Bit 4 of the id is
// folded into bit 0 (id ^ ((id >> 4) & 1)) so that the 4-byte writes of lanes
// l and l+16 use different banks; 16-byte reads of 32 consecutive ids stay
// conflict-free.
__device__ __forceinline__ int xswz(int id) { return id ^ ((id >> 4) & 1); }

// Stage b fused with the exchange writes: as soon as tiles (2v, 2v+1) are
// transformed, dword v of all 16 chunks goes to LDS (while the next tiles'
// MFMAs run).
__device__ __forceinline__ void stage_rows_and_write(f32x16 (&acc)[8], const u32x4 (&h)[2],
                                                     uint32_t* xbuf, int wbase) {
  const f32x16 zero = {};
  auto write_pair = [&](int v) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      xbuf[xswz(wbase + ((r & 7) << 5) + ((r >> 3) << 9)) * 4 + v] = pk(acc[2 * v][r], acc[2 * v + 1][r]);
  };
#pragma unroll
  for (int v = 0; v < 4; ++v) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int t = 2 * v + e;
      const u32x4 a0 = pack8(acc[t], 0), a1 = pack8(acc[t], 8);
      f32x16 d = mfma(a0, h[0], zero);
      acc[t] = mfma(a1, h[1], d);
    }
    if (v > 0) write_pair(v - 1);
  }
  write_pair(3);
}

// Stage c (data as B operand) after the exchange: all 16 operand chunks are
// read first, the MFMAs start as they arrive.
__device__ __forceinline__ void read_and_stage_c(f32x16 (&acc)[8], const u32x4 (&h)[2], const u32x4* xbuf,
                                                 int rbase) {
  __syncthreads();
  u32x4 b[8][2];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    b[t][0] = xbuf[xswz(rbase + (t << 5))];
    b[t][1] = xbuf[xswz(rbase + (t << 5) + (1 << 11))];
  }
  const f32x16 zero = {};
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    f32x16 d = mfma(h[0], b[t][0], zero);
    acc[t] = mfma(h[1], b[t][1], d);
  }
}

struct Ctx {
  int lane32, l5, wave;
  uint32_t bkey;
  uint32_t base0, base1;  // word-index bases in S0 and S1
  int wbase, rbase;       // LDS exchange chunk-id bases
};

__device__ __forceinline__ Ctx make_ctx(uint32_t seed32, int64_t block) {
  Ctx x;
  const int tid = threadIdx.x;
  x.lane32 = tid & 31;
  x.l5 = (tid >> 5) & 1;
  x.wave = tid >> 6;
  x.bkey = block_key(seed32, block);
  x.base0 = (uint32_t)(x.lane32 | (x.l5 << 5) | (x.wave << 8));
  x.base1 = (uint32_t)(x.lane32 | (x.wave << 5) | (x.l5 << 7));
  x.wbase = x.lane32 + (x.l5 << 8) + (x.wave << 10);
  x.rbase = x.lane32 + (x.wave << 8) + (x.l5 << 10);
  return x;
}

// Block position of the first of 8 consecutive elements of load/store chunk
// (t, c) in S0, or of chunk r in S1.
__device__ __forceinline__ int pos_s0(const Ctx& x, int t, int c) {
  return ((x.lane32 << 5) + (x.l5 << 10) + (x.wave << 13)) +
         (((t & 1) << 3) + (((t >> 1) & 1) << 4) + (c << 11) + ((t >> 2) << 12));
}
__device__ __forceinline__ int pos_s1(const Ctx& x, int r) {
  return ((x.lane32 << 5) + (x.wave << 10) + (x.l5 << 12)) +
         (((r & 1) << 3) + (((r >> 1) & 1) << 4) + ((r >> 2) << 13));
}

// Sign words of the layer applied after the chain, for the output layout
// (S1 when L is odd, S0 when even), optionally in the swap_idx04 pair layout.
template <int L>
__device__ __forceinline__ void final_words(const Ctx& x, int layer, uint32_t (&nw)[4], bool permute) {
  const uint32_t lkey = layer_key(layer);
  constexpr bool kOutS1 = (L % 2) == 1;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    uint32_t word;
    if (kOutS1)
      word = x.base1 | ((uint32_t)s << 8);  // s = r >> 2 (p13, p14)
    else
      word = x.base0 | ((uint32_t)(s & 1) << 6) | ((uint32_t)(s >> 1) << 7);  // s = c + 2*t2
    const uint32_t w = ~sign_word(x.bkey, lkey, word);
    nw[s] = permute ? swap_idx04(w) : w;
  }
}

// Runs the L-layer chain on a block whose unsigned input sits in `src`
// (src[t][c] = 8 bf16 of S0 chunk (t, c), loads possibly still in flight).
// sign_layer(i) is the sign layer applied before kernel layer i (i < L) and
// after the last one (i = L); the words of the latter are returned in `fin`
// (pair layout when kFinalPairs).  On return acc holds the chain's result,
// before that last sign layer, in S1 (L odd) or S0 (L even).  Uses both
// exchange buffers; xbufs[L & 1] is free again for wave-local use on return.
template <int L, bool kFinalPairs, class SignLayer>
__device__ __forceinline__ void run_chain(f32x16 (&acc)[8], const Ctx& x, u32x4 (*xbufs)[4096],
                                          const u32x4 (&src)[8][2], SignLayer sign_layer,
                                          uint32_t (&fin)[4]) {
  // Hashes and Walsh operands first: independent of the source loads.
  uint32_t nw[L][4];
#pragma unroll
  for (int i = 0; i < L; ++i) {
    if (i & 1)
      layer_words<true>(x.bkey, sign_layer(i), x.base1, nw[i]);
    else
      layer_words<false>(x.bkey, sign_layer(i), x.base0, nw[i]);
  }
  final_words<L>(x, sign_layer(L), fin, kFinalPairs);
  const int lane = threadIdx.x & 63;
  u32x4 hp4[2], hq4[2], hq8[2], hlast[2];
  walsh_operand<0, 1, 2, 3, 4>(lane, 0.25f, hp4);
  walsh_operand<0, 1, 3, 2, 4>(lane, 0.25f, hq4);
  walsh_operand<0, 1, 3, 2, 4>(lane, 0.125f, hq8);
  {
    // last stage c: plain Walsh (even last layer) or permuted (odd), scaled by 2^(-2 - L/2)
    const float s = (L == 1) ? 0.17677669529663688f : (L == 2) ? 0.125f : 0.08838834764831845f;
    if ((L - 1) % 2 == 0)
      walsh_operand<0, 1, 2, 3, 4>(lane, s, hlast);
    else
      walsh_operand<0, 1, 3, 2, 4>(lane, s, hlast);
  }
  const f32x16 zero = {};
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const bool odd = i & 1;
    if (i == 0) {
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        u32x4 a[2] = {src[t][0], src[t][1]};
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int v = 0; v < 4; ++v) a[c][v] ^= operand_mask<false>(nw[0], t, c, v);
        f32x16 d = mfma(a[0], hq4[0], zero);
        acc[t] = mfma(a[1], hq4[1], d);
      }
    } else if (odd) {
      stage_rows_signed<true>(acc, hp4, nw[i]);
    } else {
      stage_rows_signed<false>(acc, hq4, nw[i]);
    }
    // Layer i exchanges through buffer i & 1: its previous readers (layer
    // i - 2) are past layer i - 1's barrier.
    u32x4* xbuf = xbufs[i & 1];
    stage_rows_and_write(acc, hq8, reinterpret_cast<uint32_t*>(xbuf), x.wbase);
    read_and_stage_c(acc, i == L - 1 ? hlast : (odd ? hq4 : hp4), xbuf, x.rbase);
  }
}

// Raw buffer resource over `bytes` bytes at `base`: loads past the end read 0,
// stores past the end are dropped (offsets are 32-bit).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint32_t load16(__amdgpu_buffer_rsrc_t r, int elem) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, elem * 2, 0, 0);
}

// 8 bf16 at element `p` of a buffer holding `count` elements; elements at or
// past `count` read as 0.
__device__ __forceinline__ u32x4 load_chunk(__amdgpu_buffer_rsrc_t r, int p, int count) {
  u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, p * 2, 0, 0);
  if (p < count && p + 8 > count) {  // straddles the end: exact element loads
    v = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (p + e < count) v[e >> 1] |= load16(r, p + e) << (16 * (e & 1));
  }
  return v;
}

// ---------------------------------------------------------------- forward

template <int L>
__global__ __launch_bounds__(kThreads) void bfht_mfma15_fwd(const __bf16* __restrict__ latent,
                                                            __bf16* __restrict__ out, int n,
                                                            int64_t first_block, int64_t start,
                                                            int64_t stop, uint32_t seed32) {
  __shared__ u32x4 xbufs[2][4096];  // layer exchanges; xbufs[L & 1] then stages the output
  const int64_t block = first_block + blockIdx.x;
  const Ctx x = make_ctx(seed32, block);
  const auto lat_r = rsrc(latent, (uint32_t)n * 2u);
  u32x4 src[8][2];
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c) src[t][c] = load_chunk(lat_r, pos_s0(x, t, c), n);
  f32x16 acc[8];
  uint32_t nw[4];
  run_chain<L, true>(acc, x, xbufs, src, [](int i) { return i; }, nw);

  // block-local output range [lo, hi); out element of block position p is (base - start) + p
  const int64_t base = block * kB;
  const int lo = (int)(start - base > 0 ? start - base : 0);
  const int hi = (int)(stop - base < kB ? stop - base : kB);
  __bf16* oblk = out + (base - start);
  const bool full = lo == 0 && hi == kB && (((uintptr_t)oblk & 15) == 0);
  // Each wave owns whole runs of positions (S1: 1024-element runs, S0: 8192):
  // its signed bf16 chunks go through its own LDS region in position order
  // (local chunk c at c ^ ((c >> 4) & 3): conflict-free both ways) and out with
  // consecutive lanes on consecutive 16-byte chunks.  No block barrier.
  u32x4* region = xbufs[L & 1] + x.wave * 1024;
  auto put = [&](int local, u32x4 v) { region[local ^ ((local >> 4) & 3)] = v; };
  if constexpr (L % 2 == 1) {  // output in S1: chunk r packs tiles (t, t^1)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      u32x4 v;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int b = ((r >> 1) & 1) | (q << 1) | ((r & 1) << 3);
        v[q] = pk(acc[2 * q][r], acc[2 * q + 1][r]) ^ ((nw[r >> 2] << (15 - b)) & kPairSign);
      }
      put(((x.lane32 << 2) + (x.l5 << 7)) + ((r & 3) + ((r >> 2) << 8)), v);
    }
  } else {  // output in S0: chunk (t, c) packs registers 8c .. 8c+7
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        u32x4 v = pack8(acc[t], 8 * c);
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] ^= operand_mask<false>(nw, t, c, q);
        put(((x.lane32 << 2) + (x.l5 << 7)) + ((t & 1) + (((t >> 1) & 1) << 1) + (c << 8) + ((t >> 2) << 9)), v);
      }
  }
  // LDS operations of one wave complete in order; keep the compiler from
  // moving the reads above the writes.
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const auto out_r = rsrc(full ? (const void*)oblk : (const void*)out, full ? (uint32_t)(kB * 2) : 0u);
  uint16_t* oblk16 = reinterpret_cast<uint16_t*>(oblk);
  const int lane = threadIdx.x & 63;
  u32x4 v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int local = i * 64 + lane;
    v[i] = region[local ^ ((local >> 4) & 3)];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int local = i * 64 + lane;
    // local chunk -> block chunk: S1 local bits 0-6 | l5 (7) | r>>2 (8-9), wave at 7-8;
    // S0 local bits 0-9, wave at 10-11
    const int c = (L % 2 == 1)
                      ? ((local & 127) | (x.wave << 7) | (((local >> 7) & 1) << 9) | ((local >> 8) << 10))
                      : (local | (x.wave << 10));
    const int p = c * 8;
    if (full) {
      __builtin_amdgcn_raw_buffer_store_b128(v[i], out_r, p * 2, 0, 0);
    } else if (p + 8 > lo && p < hi) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (p + e >= lo && p + e < hi) oblk16[p + e] = (uint16_t)(v[i][e >> 1] >> (16 * (e & 1)));
    }
  }
}

// ---------------------------------------------------------------- backward

// Per-block partial latent gradient (float32, first n positions) of the
// adjoint chain D_0 H D_1 ... H D_L applied to grad scattered into the block.
template <int L>
__global__ __launch_bounds__(kThreads) void bfht_mfma15_bwd(const __bf16* __restrict__ grad,
                                                            float* __restrict__ partial, int n,
                                                            int64_t first_block, int64_t start,
                                                            int64_t stop, uint32_t seed32) {
  __shared__ u32x4 xbufs[2][4096];
  const int64_t slot = blockIdx.x;
  const int64_t block = first_block + slot;
  const Ctx x = make_ctx(seed32, block);
  const int64_t base = block * kB;
  const int lo = (int)(start - base > 0 ? start - base : 0);
  const int hi = (int)(stop - base < kB ? stop - base : kB);
  const __bf16* gblk = grad + (base - start);
  const bool full = lo == 0 && hi == kB && (((uintptr_t)gblk & 15) == 0);
  const auto g_r = rsrc(full ? (const void*)gblk : (const void*)grad, full ? (uint32_t)(kB * 2) : 0u);
  const uint16_t* gblk16 = reinterpret_cast<const uint16_t*>(gblk);
  auto load = [&](int t, int c) -> u32x4 {
    const int p = pos_s0(x, t, c);
    if (full) return __builtin_amdgcn_raw_buffer_load_b128(g_r, p * 2, 0, 0);
    u32x4 v = {0u, 0u, 0u, 0u};
    if (p + 8 > lo && p < hi) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (p + e >= lo && p + e < hi) v[e >> 1] |= (uint32_t)gblk16[p + e] << (16 * (e & 1));
    }
    return v;
  };
  u32x4 src[8][2];
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c) src[t][c] = load(t, c);
  f32x16 acc[8];
  uint32_t nw[4];
  run_chain<L, false>(acc, x, xbufs, src, [](int i) { return L - i; }, nw);

  float* prow = partial + slot * (int64_t)n;
  const auto p_r = rsrc(prow, (uint32_t)n * 4u);
  auto flip = [](float v, uint32_t w, int b) {
    return __uint_as_float(__float_as_uint(v) ^ ((w << (31 - b)) & 0x80000000u));
  };
  auto store = [&](int p, const float (&v)[8]) {
    if (p + 8 <= n) {
      __builtin_amdgcn_raw_buffer_store_b128(f32x4{v[0], v[1], v[2], v[3]}, p_r, p * 4, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(f32x4{v[4], v[5], v[6], v[7]}, p_r, p * 4 + 16, 0, 0);
    } else if (p < n) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (p + e < n) prow[p + e] = v[e];
    }
  };
  if constexpr (L % 2 == 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) v[t] = flip(acc[t][r], nw[r >> 2], t | ((r & 3) << 3));
      store(pos_s1(x, r), v);
    }
  } else {
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          v[j] = flip(acc[t][8 * c + j], nw[c + 2 * (t >> 2)], j | ((t & 3) << 3));
        store(pos_s0(x, t, c), v);
      }
  }
}

}  // namespace

bool mfma15_applicable(const BfhtArgs& a) {
  // 16-byte vector loads of the latent and the partial rows need aligned bases;
  // output and grad alignment is checked per block in the kernels.
  const bool aligned = ((uintptr_t)a.src % 16 == 0) && (a.work == nullptr || (uintptr_t)a.work % 16 == 0);
  return a.dtype == kBF16 && a.log_block == kLog && a.nblocks > 0 && a.n <= kB && aligned;
}

hipError_t launch_mfma15(const BfhtArgs& a, hipStream_t s, bool fwd) {
  const dim3 grid((unsigned)a.nblocks), block(kThreads);
  if (fwd) {
    auto* src = (const __bf16*)a.src;
    auto* dst = (__bf16*)a.dst;
    switch (a.layers) {
      case 1: hipLaunchKernelGGL(bfht_mfma15_fwd<1>, grid, block, 0, s, src, dst, (int)a.n, a.first_block, a.start, a.stop, a.seed32); break;
      case 2: hipLaunchKernelGGL(bfht_mfma15_fwd<2>, grid, block, 0, s, src, dst, (int)a.n, a.first_block, a.start, a.stop, a.seed32); break;
      case 3: hipLaunchKernelGGL(bfht_mfma15_fwd<3>, grid, block, 0, s, src, dst, (int)a.n, a.first_block, a.start, a.stop, a.seed32); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  auto* src = (const __bf16*)a.src;
  auto* part = (float*)a.work;
  switch (a.layers) {
    case 1: hipLaunchKernelGGL(bfht_mfma15_bwd<1>, grid, block, 0, s, src, part, (int)a.n, a.first_block, a.start, a.stop, a.seed32); break;
    case 2: hipLaunchKernelGGL(bfht_mfma15_bwd<2>, grid, block, 0, s, src, part, (int)a.n, a.first_block, a.start, a.stop, a.seed32); break;
    case 3: hipLaunchKernelGGL(bfht_mfma15_bwd<3>, grid, block, 0, s, src, part, (int)a.n, a.first_block, a.start, a.stop, a.seed32); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace lwl
