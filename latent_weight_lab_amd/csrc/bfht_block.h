// Whole-block VALU transforms (blocks of 2^0 .. 2^15 held in registers with
// LDS exchanges), shared by the per-generator kernels (bfht_kernels.hip) and
// the grouped weight-cache kernels (bfht_grouped_kernels.hip).
#pragma once

#include "bfht_device.h"
#include "bfht_launch.h"

namespace lwl {

// Element loads / stores through a raw buffer resource: element index i of the
// buffer; indices past the end read 0 / are dropped by the buffer range check,
// and negative indices are sent to the out-of-range offset 2^31 explicitly (the
// check covers only the per-lane offset, and a wrapped offset near 2^32 must
// never reach it).  Buffers stay below 2 GiB.  The resource must be uniform
// across the wave (a divergent one costs a loop over its distinct values).
constexpr uint32_t kOobOffset = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, uint64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)(bytes < 0x80000000ull ? bytes : 0x80000000ull), 0x00020000);
}
template <class T>
__device__ __forceinline__ int buf_offset(int i) {
  return (int)(i < 0 ? kOobOffset : (uint32_t)i * (uint32_t)sizeof(T));
}
template <class T>
__device__ __forceinline__ float buf_load(__amdgpu_buffer_rsrc_t r, int i) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, buf_offset<T>(i), 0, 0));
  } else {
    const uint16_t h = __builtin_amdgcn_raw_buffer_load_b16(r, buf_offset<T>(i), 0, 0);
    return to_f32(__builtin_bit_cast(T, h));
  }
}
template <class T>
__device__ __forceinline__ void buf_store(float v, __amdgpu_buffer_rsrc_t r, int i) {
  if constexpr (sizeof(T) == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, buf_offset<T>(i), 0, 1 | 16);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f32<T>(v)), r, buf_offset<T>(i), 0,
                                          1 | 16);
  }
}
// The same at element base + c with base >= 0 per lane and c a wave-uniform
// constant: c goes into the scalar offset, which the range check does not
// cover, so these are only for accesses known to be in range (whole blocks).
template <class T>
__device__ __forceinline__ float buf_load_at(__amdgpu_buffer_rsrc_t r, int base, int c) {
  const int vo = (int)((uint32_t)base * (uint32_t)sizeof(T)), so = c * (int)sizeof(T);
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0));
  } else {
    const uint16_t h = __builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0);
    return to_f32(__builtin_bit_cast(T, h));
  }
}
template <class T>
__device__ __forceinline__ void buf_store_at(float v, __amdgpu_buffer_rsrc_t r, int base, int c) {
  const int vo = (int)((uint32_t)base * (uint32_t)sizeof(T)), so = c * (int)sizeof(T);
  if constexpr (sizeof(T) == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, vo, so, 1 | 16);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f32<T>(v)), r, vo, so, 1 | 16);
  }
}
// Element base + c with base >= 0 per lane and c >= 0 constant, range-checked
// (positions past the buffer are dropped / read 0): both in the lane offset,
// where a small c folds into the instruction's immediate offset.
template <class T>
__device__ __forceinline__ void buf_store_nn(float v, __amdgpu_buffer_rsrc_t r, int base, int c) {
  const int vo = (int)((uint32_t)(base + c) * (uint32_t)sizeof(T));
  if constexpr (sizeof(T) == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, vo, 0, 1 | 16);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f32<T>(v)), r, vo, 0, 1 | 16);
  }
}

// ---------------------------------------------------------------- whole block

// Blocks of up to 2^5 (one thread holds a whole block, no LDS).
template <int LB, class T, class Store>
__device__ __forceinline__ void block_fwd_small(const T* __restrict__ latent, Store out, int n, int64_t first_block,
                                                int64_t slot, int64_t nblocks, int64_t start, int64_t stop,
                                                uint32_t seed32, int layers) {
  using Gm = Geo<LB>;
  static_assert(Gm::TB == 1, "one thread per block");
  const bool active = slot < nblocks;
  const int64_t block = first_block + (active ? slot : 0);
  const uint32_t bkey = block_key(seed32, block);
  float v[Gm::E];
  {
    const uint32_t w = sign_word(bkey, layer_key(0), 0u);
    const auto lat_r = tile_rsrc(latent, (uint64_t)n * sizeof(T));  // positions >= n read 0
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) v[r] = signed_by(buf_load<T>(lat_r, r), w, r);
  }
  const float scale = inv_sqrt_block<LB>();
  for (int layer = 0; layer < layers; ++layer) {
    butterflies<Gm::E>(v, Gm::LE);
    const uint32_t w = sign_word(bkey, layer_key(layer + 1), 0u);
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) v[r] = signed_by(v[r], w, r) * scale;
  }
  if (!active) return;
  const int64_t base = block * Gm::B;
  const int64_t lo = start - base > 0 ? start - base : 0;
  const int64_t hi = stop - base < Gm::B ? stop - base : Gm::B;
#pragma unroll
  for (int r = 0; r < Gm::E; ++r)
    if (r >= lo && r < hi) out.at(base + r - start, v[r]);
}

template <int LB, class T, class Load>
__device__ __forceinline__ void block_bwd_small(Load grad, float* __restrict__ partial, int64_t stride,
                                                T* __restrict__ grad_latent, int n, int64_t first_block, int64_t slot,
                                                int64_t nblocks, int64_t start, int64_t stop, uint32_t seed32,
                                                int layers, int direct) {
  using Gm = Geo<LB>;
  static_assert(Gm::TB == 1, "one thread per block");
  const bool active = slot < nblocks;
  const int64_t block = first_block + (active ? slot : 0);
  const uint32_t bkey = block_key(seed32, block);
  const int64_t base = block * Gm::B;
  const int64_t lo = start - base > 0 ? start - base : 0;
  const int64_t hi = stop - base < Gm::B ? stop - base : Gm::B;
  // every lane is a different block: element loads from a valid index (the
  // slice's first element stands in for positions outside it), then a select
  float v[Gm::E];
#pragma unroll
  for (int r = 0; r < Gm::E; ++r) {
    const bool valid = active && r >= lo && r < hi;
    const float x = grad.at(valid ? base + r - start : 0);
    v[r] = valid ? x : 0.0f;
  }
  const float scale = inv_sqrt_block<LB>();
  for (int layer = layers - 1; layer >= 0; --layer) {
    const uint32_t w = sign_word(bkey, layer_key(layer + 1), 0u);
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) v[r] = signed_by(v[r], w, r);
    butterflies<Gm::E>(v, Gm::LE);
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) v[r] *= scale;
  }
  if (!active) return;
  const uint32_t w0 = sign_word(bkey, layer_key(0), 0u);
#pragma unroll
  for (int r = 0; r < Gm::E; ++r) {
    if (r < n) {
      const float g = signed_by(v[r], w0, r);
      if (direct)
        grad_latent[r] = from_f32<T>(g);
      else
        partial[slot * stride + r] = g;
    }
  }
}

// Layout of bit group [lo, lo + nb) (nb <= 5) in the whole-block kernels:
// register r of thread t holds position bpos(t, r, lo, nb).  The 5 register
// bits sit at position bits lo .. lo + 4 — the group's nb bits first, then
// 5 - nb bits that the group leaves untransformed — and the thread bits fill
// the other position bits from 0 up.  For a group at bit 5 or above, lanes 0-31
// then hold 32 consecutive positions, and every layout with lo >= 5 or lo = 0
// puts thread bits 6 and up on the same position bits, so an exchange between
// such layouts stays inside each wave.
template <int LB>
__host__ __device__ constexpr int bpos(int t, int r, int lo, int nb) {
  return ((t >> lo) << (lo + 5)) | (r << lo) | (t & ((1 << lo) - 1));
}
template <int LB>
__device__ __forceinline__ int bslot_base(int t, int lo, int nb) {  // padded LDS slot of (t, 0)
  return lds_index(bpos<LB>(t, 0, lo, nb));
}
template <int LB>
__device__ __forceinline__ int bslot(int base, int r, int lo, int nb) {  // slot of (t, r): disjoint bit fields
  return base + lds_index(bpos<LB>(0, r, lo, nb));
}

// Blocks of 2^6 .. 2^15: 32 values per thread.  The transform is a sequence of
// bit groups — the top group (position bits LB-5 .. LB-1, which the registers
// of the coalesced layout span: register r of thread t holds position
// r * TB + t) and groups of up to 5 bits from bit 0 up — with one LDS exchange
// between consecutive groups.  Even layers run the groups in that order, odd
// layers in reverse, so a layer boundary needs no exchange: the sign layer
// between them is applied in whatever layout the data is in, from a table of
// the block's inverted sign words in LDS (hashed once per block, one word per
// thread and layer).  The block is read and written in the coalesced layout
// (or, after an odd number of layers, in the last group's layout when that
// keeps 32 consecutive positions per half wave).  Layouts: bpos above.
template <int LB>
struct BlockSeq {
  static constexpr int TOP = LB - 5;
  static constexpr int N = 1 + (TOP + 4) / 5;  // groups
  __host__ __device__ static constexpr int lo(int g) { return g == 0 ? TOP : 5 * (g - 1); }
  __host__ __device__ static constexpr int nb(int g) {
    return g == 0 ? 5 : (TOP - 5 * (g - 1) < 5 ? TOP - 5 * (g - 1) : 5);
  }
  // the last group's layout stores 32 consecutive positions per half wave
  static constexpr bool kLastStores = lo(N - 1) >= 5;
};

constexpr int kSignTableLayers = 4;  // layers 0..3

template <int LB>
struct BlockLds {
  using Gm = Geo<LB>;
  // per block: the padded exchange buffer, then the sign-word table
  static constexpr int FLOATS = Gm::NG > 1 ? Gm::G * (Gm::PADDED + kSignTableLayers * Gm::TB) : 1;
  __device__ static float* data(float* smem, int gi) { return smem + gi * Gm::PADDED; }
  __device__ static uint32_t* table(float* smem, int gi) {
    return reinterpret_cast<uint32_t*>(smem) + table_word(gi);
  }
  // word index of group gi's table from the start of smem
  __device__ static int table_word(int gi) { return Gm::G * Gm::PADDED + gi * kSignTableLayers * Gm::TB; }
};

// Whether the exchange between groups 1 (bits 0-4) and 2 keeps every value in
// its wave.  bpos is a bit permutation of (thread, register), so it does
// when every wave-index bit of the thread (bit 6 and up) lands on the same
// position bit in both layouts: thread bit k >= 5 is position bit k + 5 in
// both, so it holds from 2^12 (two waves per block) to 2^15; below 2^12 a
// block sits in one wave anyway.
template <int LB>
constexpr bool intra_wave_pair() {
  using S = BlockSeq<LB>;
  if (S::N != 3 || Geo<LB>::TB < 64) return false;
  for (int k = 6; (1 << k) < Geo<LB>::TB; ++k)
    if (bpos<LB>(1 << k, 0, S::lo(1), S::nb(1)) != bpos<LB>(1 << k, 0, S::lo(2), S::nb(2)))
      return false;
  return true;
}
static_assert(intra_wave_pair<15>() && intra_wave_pair<14>() && intra_wave_pair<13>() && intra_wave_pair<12>() &&
                  !intra_wave_pair<10>(),
              "intra-wave exchange pairs");
static_assert(bpos<15>(1000, 7, 10, 5) == 7 * 1024 + 1000 && bpos<13>(5, 3, 8, 5) == 3 * 256 + 5,
              "the top group's layout is the coalesced one: register r of thread t at r * TB + t");

// Register exchange from group layout (lo_a, nb_a) to (lo_b, nb_b) through LDS.
// Position p always sits in slot lds_index(p), so a thread writes exactly the
// slots it read in the previous exchange, which no other thread reads in
// between: the writes need no barrier before them.  The reads need every
// thread's writes done (a barrier), except when the exchange keeps each value
// in its wave (`intra_wave`): a wave's LDS accesses are performed in order.
template <int LB>
__device__ __forceinline__ void exchange(float (&v)[32], float* lds, int t, int lo_a, int nb_a, int lo_b, int nb_b,
                                         bool intra_wave = false) {
  const int wb = bslot_base<LB>(t, lo_a, nb_a);
#pragma unroll
  for (int r = 0; r < 32; ++r) lds[bslot<LB>(wb, r, lo_a, nb_a)] = v[r];
  if (intra_wave)
    asm volatile("" ::: "memory");  // keep the reads after the writes
  else
    __syncthreads();
  const int rb = bslot_base<LB>(t, lo_b, nb_b);
#pragma unroll
  for (int r = 0; r < 32; ++r) v[r] = lds[bslot<LB>(rb, r, lo_b, nb_b)];
}

// x with its sign bit XOR-ed with bit 31 of m (one v_bitop3).
__device__ __forceinline__ float flip_by_msb(float x, uint32_t m) {
  return __uint_as_float(__float_as_uint(x) ^ (m & 0x80000000u));
}

// Sign layer in layout (lo, nb): v[r] negated where the bit of its position is
// set in the layer's flip table (word p >> 5, bit p & 31; the table holds the
// sign words inverted), as an XOR of the float's sign bit.  Position = per-thread
// base OR a per-register constant (disjoint bits), so word index and bit split
// the same way.  When the group starts at bit 5 or above, every register's bit
// is the thread's base & 31, and the words of two registers are shifted
// together by one 64-bit shift (each dword's bit 31 is its own word's bit: the
// low word's bits shifted into the high dword stay below bit 31).  The
// 2^(-LB/2) of every layer is applied once, at the end (transform_scale).
template <int LB>
__device__ __forceinline__ void sign_flip(float (&v)[32], const uint32_t* smem_words, int table, int t, int lo,
                                          int nb) {
  const int base = bpos<LB>(t, 0, lo, nb);
  // The table sits above the exchange buffer (beyond the 64 KiB the LDS
  // instructions' offset field reaches): its index is opaque to the compiler,
  // so it is added once and the per-register word offsets fold into the reads.
  int first = table + (base >> 5);
  asm("" : "+v"(first));
  const uint32_t* flips = smem_words + first - (base >> 5);
  if (lo >= 5) {
    const uint32_t s = 31u - (uint32_t)(base & 31);
#pragma unroll
    for (int r = 0; r < 32; r += 2) {
      const int c0 = bpos<LB>(0, r, lo, nb), c1 = bpos<LB>(0, r + 1, lo, nb);
      const uint64_t pair = (uint64_t)flips[(base >> 5) + (c0 >> 5)] |
                            ((uint64_t)flips[(base >> 5) + (c1 >> 5)] << 32);
      uint64_t m;
      asm("v_lshlrev_b64 %0, %1, %2" : "=v"(m) : "v"(s), "v"(pair));
      v[r] = flip_by_msb(v[r], (uint32_t)m);
      v[r + 1] = flip_by_msb(v[r + 1], (uint32_t)(m >> 32));
    }
  } else {
#pragma unroll
    for (int r = 0; r < 32; ++r) {
      const int c = bpos<LB>(0, r, lo, nb);
      const int bit = (base & 31) | (c & 31);
      v[r] = flip_by_msb(v[r], flips[(base >> 5) + (c >> 5)] << (31 - bit));
    }
  }
}

// 2^(-LB * layers / 2): the normalization of `layers` transforms of order 2^LB,
// exact but for one rounding of 1/sqrt(2) when LB * layers is odd.
template <int LB>
__device__ __forceinline__ float transform_scale(int layers) {
  const int e = LB * layers;
  const float p2 = __builtin_ldexpf(1.0f, -(e >> 1));
  return (e & 1) ? 0.70710678118654752440f * p2 : p2;
}

// One layer's transform (unnormalized), groups forward (even layers: top first,
// ending in the last group's layout) or reversed (odd layers).
template <int LB>
__device__ __forceinline__ void layer_fht(float (&v)[32], float* lds, int t, bool reversed) {
  using S = BlockSeq<LB>;
  constexpr bool kOneWave = Geo<LB>::TB <= 64;  // a block in one wave: its exchanges stay there
  constexpr bool kIntra12 = intra_wave_pair<LB>();
  if (!reversed) {
    butterflies<32>(v, S::nb(0));
#pragma unroll
    for (int g = 1; g < S::N; ++g) {
      exchange<LB>(v, lds, t, S::lo(g - 1), S::nb(g - 1), S::lo(g), S::nb(g), kOneWave || (kIntra12 && g == 2));
      butterflies<32>(v, S::nb(g));
    }
  } else {
    butterflies<32>(v, S::nb(S::N - 1));
#pragma unroll
    for (int g = S::N - 2; g >= 0; --g) {
      exchange<LB>(v, lds, t, S::lo(g + 1), S::nb(g + 1), S::lo(g), S::nb(g), kOneWave || (kIntra12 && g == 1));
      butterflies<32>(v, S::nb(g));
    }
  }
}

// Flip table: the block's sign words of layers 0..layers, inverted (a set bit
// negates its position), one word per thread and layer.
template <int LB>
__device__ __forceinline__ void fill_sign_table(uint32_t* tab, uint32_t bkey, int t, int layers) {
  for (int l = 0; l <= layers; ++l) tab[l * Geo<LB>::TB + t] = ~sign_word(bkey, layer_key(l), (uint32_t)t);
}

// Forward of block slot `slot` (block first_block + slot of one generator) by
// thread group gi of the workgroup; every thread of the workgroup calls it
// (barriers inside), threads of an inactive slot (slot >= nblocks) included.
template <int LB, class T, class Store>
__device__ __forceinline__ void block_fwd_slot(const T* __restrict__ latent, Store out, int n,
                                               int64_t first_block, int64_t slot, int64_t nblocks, int64_t start,
                                               int64_t stop, uint32_t seed32, int layers, float* smem) {
  using Gm = Geo<LB>;
  using S = BlockSeq<LB>;
  if constexpr (Gm::NG <= 1) {  // B <= 2^5
    block_fwd_small<LB, T>(latent, out, n, first_block, slot, nblocks, start, stop, seed32, layers);
  } else {
    const int gi = threadIdx.x >> Gm::LT;
    const int t = threadIdx.x & (Gm::TB - 1);
    const bool active = slot < nblocks;
    const int64_t block = first_block + (active ? slot : 0);
    float* lds = BlockLds<LB>::data(smem, gi);
    uint32_t* tab = BlockLds<LB>::table(smem, gi);
    fill_sign_table<LB>(tab, block_key(seed32, block), t, layers);
    // coalesced layout: register r of thread t holds position r * TB + t;
    // positions >= n read 0 (buffer range)
    const auto lat_r = tile_rsrc(latent, (uint64_t)n * sizeof(T));
    float v[32];
    if (n >= Gm::B) {  // every position in range: register offsets in the scalar offset
#pragma unroll
      for (int r = 0; r < 32; ++r) v[r] = buf_load_at<T>(lat_r, t, r * Gm::TB);
    } else {
#pragma unroll
      for (int r = 0; r < 32; ++r) v[r] = buf_load<T>(lat_r, r * Gm::TB + t);
    }
    __syncthreads();  // the sign table is complete
    const uint32_t* words = reinterpret_cast<const uint32_t*>(smem);
    const int tw = BlockLds<LB>::table_word(gi);
    sign_flip<LB>(v, words, tw, t, S::lo(0), S::nb(0));
    for (int layer = 0; layer < layers; ++layer) {
      const bool odd = layer & 1;
      layer_fht<LB>(v, lds, t, odd);
      if (odd)
        sign_flip<LB>(v, words, tw + (layer + 1) * Gm::TB, t, S::lo(0), S::nb(0));
      else
        sign_flip<LB>(v, words, tw + (layer + 1) * Gm::TB, t, S::lo(S::N - 1), S::nb(S::N - 1));
    }
    const float scale = transform_scale<LB>(layers);
    // store from the layout the last layer ended in
    const int64_t base = block * Gm::B;
    const int64_t lo = start - base > 0 ? start - base : 0;
    const int64_t hi = stop - base < Gm::B ? stop - base : Gm::B;
    auto store = [&](int glo, int gnb) {
      if (!active) return;
      const int pb = bpos<LB>(t, 0, glo, gnb);
      if constexpr (Gm::TB >= 64) {
        // one block per wave: a uniform buffer resource over the block's range,
        // positions outside [lo, hi) dropped by its range check; a whole block
        // (the wave-uniform common case) stores without per-element checks
        const auto out_r = out.range(base + lo - start, hi - lo);
        if (lo == 0 && hi == Gm::B) {
#pragma unroll
          for (int r = 0; r < 32; ++r) out.whole(out_r, pb, bpos<LB>(0, r, glo, gnb), v[r] * scale);
        } else {
#pragma unroll
          for (int r = 0; r < 32; ++r) out(out_r, pb + bpos<LB>(0, r, glo, gnb) - (int)lo, v[r] * scale);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 32; ++r) {
          const int p = pb | bpos<LB>(0, r, glo, gnb);
          if (p >= lo && p < hi) out.at(base + p - start, v[r] * scale);
        }
      }
    };
    if (!(layers & 1)) {
      store(S::lo(0), S::nb(0));
    } else if constexpr (S::kLastStores) {
      store(S::lo(S::N - 1), S::nb(S::N - 1));
    } else {
      exchange<LB>(v, lds, t, S::lo(S::N - 1), S::nb(S::N - 1), S::lo(0), S::nb(0), Gm::TB <= 64);
      store(S::lo(0), S::nb(0));
    }
  }
}

// Backward: adjoint chain D_0 H D_1 ... H D_L on grad scattered into the block.
// Writes partial[slot * stride + p] (float32) for p < n, or the final gradient
// in T when `direct` (a single block).
template <int LB, class T, class Load>
__device__ __forceinline__ void block_bwd_slot(Load grad, float* __restrict__ partial, int64_t stride,
                                               T* __restrict__ grad_latent, int n, int64_t first_block, int64_t slot,
                                               int64_t nblocks, int64_t start, int64_t stop, uint32_t seed32,
                                               int layers, int direct, float* smem) {
  using Gm = Geo<LB>;
  using S = BlockSeq<LB>;
  if constexpr (Gm::NG <= 1) {  // B <= 2^5
    block_bwd_small<LB, T>(grad, partial, stride, grad_latent, n, first_block, slot, nblocks, start, stop, seed32,
                           layers, direct);
  } else {
    const int gi = threadIdx.x >> Gm::LT;
    const int t = threadIdx.x & (Gm::TB - 1);
    const bool active = slot < nblocks;
    const int64_t block = first_block + (active ? slot : 0);
    float* lds = BlockLds<LB>::data(smem, gi);
    uint32_t* tab = BlockLds<LB>::table(smem, gi);
    fill_sign_table<LB>(tab, block_key(seed32, block), t, layers);
    const int64_t base = block * Gm::B;
    const int64_t lo = start - base > 0 ? start - base : 0;
    const int64_t hi = stop - base < Gm::B ? stop - base : Gm::B;
    // positions outside [lo, hi), and every position of an inactive slot, read 0
    float v[32];
    if constexpr (Gm::TB >= 64) {
      const auto g_r = grad.range(base + lo - start, active ? hi - lo : 0);
      if (active && lo == 0 && hi == Gm::B) {  // a whole block: no per-element checks
#pragma unroll
        for (int r = 0; r < 32; ++r) v[r] = grad.whole(g_r, t, r * Gm::TB);
      } else {
#pragma unroll
        for (int r = 0; r < 32; ++r) v[r] = grad(g_r, r * Gm::TB + t - (int)lo);
      }
    } else {
      // several blocks per wave: element loads from a valid index (the slice's
      // first element stands in for positions outside it), then a select
#pragma unroll
      for (int r = 0; r < 32; ++r) {
        const int p = r * Gm::TB + t;
        const bool valid = active && p >= lo && p < hi;
        const float x = grad.at(valid ? base + p - start : 0);
        v[r] = valid ? x : 0.0f;
      }
    }
    __syncthreads();  // the sign table is complete
    const uint32_t* words = reinterpret_cast<const uint32_t*>(smem);
    const int tw = BlockLds<LB>::table_word(gi);
    sign_flip<LB>(v, words, tw + layers * Gm::TB, t, S::lo(0), S::nb(0));
    for (int i = 0; i < layers; ++i) {
      const bool odd = i & 1;
      layer_fht<LB>(v, lds, t, odd);
      const int lw = tw + (layers - 1 - i) * Gm::TB;
      if (odd)
        sign_flip<LB>(v, words, lw, t, S::lo(0), S::nb(0));
      else
        sign_flip<LB>(v, words, lw, t, S::lo(S::N - 1), S::nb(S::N - 1));
    }
    const float scale = transform_scale<LB>(layers);
    auto write = [&](int glo, int gnb) {
      if (!active) return;
      const int pb = bpos<LB>(t, 0, glo, gnb);
      if constexpr (Gm::TB >= 64) {
        // one block per wave: uniform resources, positions >= n dropped
        const auto d_r = direct ? tile_rsrc(grad_latent, (uint64_t)n * sizeof(T))
                                : tile_rsrc(partial + slot * stride, (uint64_t)n * 4);
#pragma unroll
        for (int r = 0; r < 32; ++r) {
          const int c = bpos<LB>(0, r, glo, gnb);  // disjoint from pb's bits
          if (direct)
            buf_store_nn<T>(v[r] * scale, d_r, pb, c);
          else
            buf_store_nn<float>(v[r] * scale, d_r, pb, c);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 32; ++r) {
          const int p = pb | bpos<LB>(0, r, glo, gnb);
          if (p < n) {
            if (direct)
              grad_latent[p] = from_f32<T>(v[r] * scale);
            else
              partial[slot * stride + p] = v[r] * scale;
          }
        }
      }
    };
    if (!(layers & 1)) {
      write(S::lo(0), S::nb(0));
    } else if constexpr (S::kLastStores) {
      write(S::lo(S::N - 1), S::nb(S::N - 1));
    } else {
      exchange<LB>(v, lds, t, S::lo(S::N - 1), S::nb(S::N - 1), S::lo(0), S::nb(0), Gm::TB <= 64);
      write(S::lo(0), S::nb(0));
    }
  }
}

// Rounding of a float32 value to T and back.
template <class T>
__device__ __forceinline__ float round_to(float v) {
  return to_f32(from_f32<T>(v));
}

}  // namespace lwl
