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

// Data as A operand: acc[t] <- (packed acc[t]) x H, for all 8 tiles.
__device__ __forceinline__ void stage_rows(f32x16 (&acc)[8], const u32x4 (&h)[2]) {
  const f32x16 zero = {};
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const u32x4 a0 = pack8(acc[t], 0), a1 = pack8(acc[t], 8);
    f32x16 d = mfma(a0, h[0], zero);
    acc[t] = mfma(a1, h[1], d);
  }
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

// LDS exchange + stage c (data as B operand).  Chunk id of 8 packed values:
// write side lane32 | (r&7)<<5 | l5<<8 | (r>>3)<<9 | wave<<10 (8 tiles packed),
// read side lane32 | t<<5 | wave<<8 | l5<<10 | c<<11.
__device__ __forceinline__ void exchange_and_stage_c(f32x16 (&acc)[8], const u32x4 (&h)[2], u32x4* lds,
                                                     int lane32, int l5, int wave) {
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    u32x4 chunk;
    chunk[0] = pk(acc[0][r], acc[1][r]);
    chunk[1] = pk(acc[2][r], acc[3][r]);
    chunk[2] = pk(acc[4][r], acc[5][r]);
    chunk[3] = pk(acc[6][r], acc[7][r]);
    lds[lane32 | ((r & 7) << 5) | (l5 << 8) | ((r >> 3) << 9) | (wave << 10)] = chunk;
  }
  __syncthreads();
  const f32x16 zero = {};
  const int rbase = lane32 | (wave << 8) | (l5 << 10);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const u32x4 b0 = lds[rbase | (t << 5)];
    const u32x4 b1 = lds[rbase | (t << 5) | (1 << 11)];
    f32x16 d = mfma(h[0], b0, zero);
    acc[t] = mfma(h[1], b1, d);
  }
}

struct Ctx {
  int lane32, l5, wave;
  uint32_t bkey;
  uint32_t base0, base1;  // word-index bases in S0 and S1
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
  return x;
}

// Block position of the first of 8 consecutive elements of load/store chunk
// (t, c) in S0, or of chunk r in S1.
__device__ __forceinline__ int pos_s0(const Ctx& x, int t, int c) {
  return ((t & 1) << 3) | (((t >> 1) & 1) << 4) | (x.lane32 << 5) | (x.l5 << 10) | (c << 11) |
         ((t >> 2) << 12) | (x.wave << 13);
}
__device__ __forceinline__ int pos_s1(const Ctx& x, int r) {
  return ((r & 1) << 3) | (((r >> 1) & 1) << 4) | (x.lane32 << 5) | (x.wave << 10) | (x.l5 << 12) |
         ((r >> 2) << 13);
}

// Runs the L-layer chain on a block whose signed-input operands are produced by
// `load(t, c)` (8 bf16 of S0 chunk (t, c), unsigned).  sign_layer(i) gives the
// sign layer applied before kernel layer i (i = 0..L-1) and after the last (i = L).
// On return acc holds the unsigned-by-final-layer result in S1 (L odd) or S0 (L even),
// scaled by the full normalization.
template <int L, class Load, class SignLayer>
__device__ __forceinline__ void run_chain(f32x16 (&acc)[8], const Ctx& x, u32x4* lds, Load load,
                                          SignLayer sign_layer) {
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
      uint32_t nw[4];
      layer_words<false>(x.bkey, sign_layer(0), x.base0, nw);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        u32x4 a[2] = {load(t, 0), load(t, 1)};
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int v = 0; v < 4; ++v) a[c][v] ^= operand_mask<false>(nw, t, c, v);
        f32x16 d = mfma(a[0], hq4[0], zero);
        acc[t] = mfma(a[1], hq4[1], d);
      }
    } else if (odd) {
      uint32_t nw[4];
      layer_words<true>(x.bkey, sign_layer(i), x.base1, nw);
      stage_rows_signed<true>(acc, hp4, nw);
    } else {
      uint32_t nw[4];
      layer_words<false>(x.bkey, sign_layer(i), x.base0, nw);
      stage_rows_signed<false>(acc, hq4, nw);
    }
    stage_rows(acc, hq8);
    if (i == L - 1)
      exchange_and_stage_c(acc, hlast, lds, x.lane32, x.l5, x.wave);
    else
      exchange_and_stage_c(acc, odd ? hq4 : hp4, lds, x.lane32, x.l5, x.wave);
  }
}

// Final sign words (swap_idx04 layout) for the output layout.
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

template <class T>
__device__ __forceinline__ u32x4 load8(const T* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// ---------------------------------------------------------------- forward

template <int L>
__global__ __launch_bounds__(kThreads) void bfht_mfma15_fwd(const __bf16* __restrict__ latent,
                                                            __bf16* __restrict__ out, int n,
                                                            int64_t first_block, int64_t start,
                                                            int64_t stop, uint32_t seed32) {
  __shared__ u32x4 lds[4096];
  const int64_t block = first_block + blockIdx.x;
  const Ctx x = make_ctx(seed32, block);
  const uint16_t* lat16 = reinterpret_cast<const uint16_t*>(latent);
  auto load = [&](int t, int c) -> u32x4 {
    const int p = pos_s0(x, t, c);
    if (p + 8 <= n) return load8(latent + p);
    u32x4 r = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (p + e < n) r[e >> 1] |= (uint32_t)lat16[p + e] << (16 * (e & 1));
    return r;
  };
  f32x16 acc[8];
  run_chain<L>(acc, x, lds, load, [](int i) { return i; });

  uint32_t nw[4];
  final_words<L>(x, L, nw, true);
  const int64_t base = block * kB;
  const bool aligned = ((start & 7) == 0);
  uint16_t* out16 = reinterpret_cast<uint16_t*>(out);
  auto store = [&](int p, u32x4 v) {
    const int64_t g = base + p;
    if (aligned && g >= start && g + 8 <= stop) {
      *reinterpret_cast<u32x4*>(out + (g - start)) = v;
    } else if (g + 8 > start && g < stop) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (g + e >= start && g + e < stop) out16[g + e - start] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
    }
  };
  if constexpr (L % 2 == 1) {  // output in S1: chunk r packs tiles (t, t^1)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      u32x4 v;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int b = ((r >> 1) & 1) | (q << 1) | ((r & 1) << 3);
        v[q] = pk(acc[2 * q][r], acc[2 * q + 1][r]) ^ ((nw[r >> 2] << (15 - b)) & kPairSign);
      }
      store(pos_s1(x, r), v);
    }
  } else {  // output in S0: chunk (t, c) packs registers 8c .. 8c+7
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        u32x4 v = pack8(acc[t], 8 * c);
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] ^= operand_mask<false>(nw, t, c, q);
        store(pos_s0(x, t, c), v);
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
  __shared__ u32x4 lds[4096];
  const int64_t slot = blockIdx.x;
  const int64_t block = first_block + slot;
  const Ctx x = make_ctx(seed32, block);
  const int64_t base = block * kB;
  const bool aligned = ((start & 7) == 0);
  const uint16_t* g16 = reinterpret_cast<const uint16_t*>(grad);
  auto load = [&](int t, int c) -> u32x4 {
    const int64_t g = base + pos_s0(x, t, c);
    if (aligned && g >= start && g + 8 <= stop) return load8(grad + (g - start));
    u32x4 r = {0u, 0u, 0u, 0u};
    if (g + 8 > start && g < stop) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (g + e >= start && g + e < stop) r[e >> 1] |= (uint32_t)g16[g + e - start] << (16 * (e & 1));
    }
    return r;
  };
  f32x16 acc[8];
  run_chain<L>(acc, x, lds, load, [](int i) { return L - i; });

  uint32_t nw[4];
  final_words<L>(x, 0, nw, false);
  float* prow = partial + slot * (int64_t)n;
  auto flip = [](float v, uint32_t w, int b) {
    return __uint_as_float(__float_as_uint(v) ^ ((w << (31 - b)) & 0x80000000u));
  };
  auto store = [&](int p, const float (&v)[8]) {
    if (p + 8 <= n) {
      *reinterpret_cast<f32x4*>(prow + p) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4*>(prow + p + 4) = f32x4{v[4], v[5], v[6], v[7]};
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
  // 16-byte vector loads/stores of the latent, grad and output need aligned bases.
  const bool aligned = ((uintptr_t)a.src % 16 == 0) && ((uintptr_t)a.dst % 16 == 0);
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
