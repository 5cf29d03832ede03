// Device building blocks shared by the BlockFHT kernels (gfx950, wave64).
//
// Sign hash: lowbias32 avalanche over (seed, block, layer, word), one 32-bit
// word per 32 positions; bit p&31 of word p>>5 set means +1
// (reference latent_weight_lab/block_fht.py:36-81, csrc/block_fht_ext_cuda.cu:27-48).
//
// Register-resident FHT: a thread holds E = 2^LE elements in VGPRs.  A "bit
// group" is a run of up to 5 index bits; for one group the thread holds the
// 2^nb elements that differ only in those bits (times 2^(LE-nb) independent
// columns), so the radix-2^nb butterflies of that group run entirely in
// registers.  Groups are exchanged through LDS with one padding float per 32
// (lds index p + p/32), which keeps every group access pattern below free of
// bank conflicts for the 64 lanes of a wave.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lwl {

typedef _Float16 f16;
typedef __bf16 bf16;

constexpr int kTileLog = 15;  // 2^15 fp32 = 128 KiB: the largest block one workgroup holds in LDS
constexpr int kMaxLog = 23;   // largest block size (after padding)

__device__ __forceinline__ uint32_t lowbias32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// seed32 ^ golden(block): constant per generated block.
__device__ __forceinline__ uint32_t block_key(uint32_t seed32, int64_t block) {
  return seed32 ^ (0x9e3779b9u * (uint32_t)(uint64_t)(block + 1));
}
__device__ __forceinline__ uint32_t layer_key(int layer) { return 0x85ebca6bu * (uint32_t)(layer + 1); }
__device__ __forceinline__ uint32_t sign_word(uint32_t bkey, uint32_t lkey, uint32_t word) {
  return lowbias32(bkey ^ lkey ^ (0xc2b2ae35u * (word + 1u)));
}

// x * (bit `bit` of `word` ? +1 : -1), as a sign-bit xor.
__device__ __forceinline__ float signed_by(float x, uint32_t word, int bit) {
  uint32_t flip = ((~word) >> bit) & 1u;
  return __uint_as_float(__float_as_uint(x) ^ (flip << 31));
}

// Sign of block position p (hash per element; for passes whose layout does not
// keep 32 consecutive positions in one thread).
__device__ __forceinline__ float signed_at(float x, uint32_t bkey, uint32_t lkey, uint32_t p) {
  return signed_by(x, sign_word(bkey, lkey, p >> 5), p & 31);
}

template <class T>
__device__ __forceinline__ float to_f32(T v) {
  return (float)v;
}
template <class T>
__device__ __forceinline__ T from_f32(float v) {
  return (T)v;
}

__device__ __forceinline__ int lds_index(int p) { return p + (p >> 5); }

// The fused linear's epilogue (lwl_bfht_linear_forward_ex) after the product v:
// + the row-sum term, + base, + bias, each a float32 add in that order and none
// contracted into an FMA, so every kernel that stores an output rounds alike.
// Absent terms are skipped rather than added as 0 (which turns -0 into +0).
__device__ __forceinline__ float linear_epilogue(float v, bool has_xs, float xs, bool has_base, float base,
                                                 bool has_bias, float bias) {
#pragma clang fp contract(off)
  if (has_xs) v = v + xs;
  if (has_base) v = v + base;
  if (has_bias) v = v + bias;
  return v;
}

// Job of workgroup `wg` in a grouped launch (uniform across the workgroup):
// the table's prefix sums count workgroups, so each workgroup serves one job.
template <class Table>
__device__ __forceinline__ int group_job(const Table& g, int wg) {
  int j = 0;
  while (j + 1 < g.count && wg >= g.prefix[j + 1]) ++j;
  return j;
}

// Index of the element that thread t holds in register r for bit group
// [lo, lo + nb) of an LB-bit index space, with 2^LE registers per thread.
// Register bits below nb walk the group; the remaining register bits pick one
// of 2^(LE-nb) columns placed above the thread index, so that for a fixed
// register the lanes of a wave touch consecutive columns.
template <int LB, int LE>
__host__ __device__ constexpr int group_pos(int t, int r, int lo, int nb) {
  const int rlo = r & ((1 << nb) - 1);
  const int c = ((r >> nb) << (LB - LE)) | t;
  return ((c >> lo) << (lo + nb)) | (rlo << lo) | (c & ((1 << lo) - 1));
}

// Unnormalized radix-2 butterflies over register-index bits [0, nb), nb <= 6.
template <int E>
__device__ __forceinline__ void butterflies(float (&v)[E], int nb) {
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    if (j < nb) {
#pragma unroll
      for (int r = 0; r < E; ++r) {
        if (!(r & (1 << j)) && (r | (1 << j)) < E) {
          const float a = v[r], b = v[r | (1 << j)];
          v[r] = a + b;
          v[r | (1 << j)] = a - b;
        }
      }
    }
  }
}

// Padded LDS index of group_pos(t, r, lo, nb): the position is a bit field of
// t OR-ed with a disjoint bit field of r, and lds_index of such a sum splits
// (their low 5 bits cannot carry), so it is a per-thread base plus a term that
// is a compile-time constant once lo, nb and r are.
template <int LB, int LE>
__device__ __forceinline__ int group_lds(int base, int r, int lo, int nb) {
  return base + lds_index(group_pos<LB, LE>(0, r, lo, nb));
}
template <int LB, int LE>
__device__ __forceinline__ int group_base(int t, int lo, int nb) {
  return lds_index(group_pos<LB, LE>(t, 0, lo, nb));
}

// Full unnormalized transform of an LB-bit block held in the coalesced layout
// (thread t, register r holds position r * 2^(LB-LE) + t, so a warp's lanes
// touch consecutive positions for every register), left in the same layout.
// The registers already span the top LE bits, so the transform starts there and
// needs one LDS exchange per remaining group of up to 5 bits plus one back to
// the coalesced layout.  All threads of the workgroup must call it.  Position p
// keeps slot lds_index(p) in every layout, so a thread's writes go to slots it
// read itself in the previous exchange (or in the previous call's last one):
// only the reads wait at a barrier.
// When the block's 2^(LB-LE) threads sit in one wave (kOneWave), the reads
// need no barrier either: a wave's LDS accesses are performed in order.
template <int LB, int LE, bool kOneWave = false>
__device__ __forceinline__ void fht_coalesced(float (&v)[1 << LE], float* lds, int t) {
  constexpr int E = 1 << LE;
  constexpr int TOP = LB - LE;  // position bits [TOP, LB) are the register bits
  static_assert(!kOneWave || (1 << TOP) <= 64, "one wave holds the block");
  auto sync = [] {
    if constexpr (kOneWave)
      asm volatile("" ::: "memory");
    else
      __syncthreads();
  };
  butterflies<E>(v, LE);
  if constexpr (TOP > 0) {
    constexpr int NR = (TOP + 4) / 5;
    int lo_cur = TOP, nb_cur = LE;
#pragma unroll
    for (int g = 0; g < NR; ++g) {
      const int lo = 5 * g, nb = (TOP - lo < 5) ? TOP - lo : 5;
      const int wb = group_base<LB, LE>(t, lo_cur, nb_cur);
#pragma unroll
      for (int r = 0; r < E; ++r) lds[group_lds<LB, LE>(wb, r, lo_cur, nb_cur)] = v[r];
      sync();
      const int rb = group_base<LB, LE>(t, lo, nb);
#pragma unroll
      for (int r = 0; r < E; ++r) v[r] = lds[group_lds<LB, LE>(rb, r, lo, nb)];
      butterflies<E>(v, nb);
      lo_cur = lo;
      nb_cur = nb;
    }
    const int wb = group_base<LB, LE>(t, lo_cur, nb_cur);
#pragma unroll
    for (int r = 0; r < E; ++r) lds[group_lds<LB, LE>(wb, r, lo_cur, nb_cur)] = v[r];
    sync();
    const int rb = group_base<LB, LE>(t, TOP, LE);
#pragma unroll
    for (int r = 0; r < E; ++r) v[r] = lds[group_lds<LB, LE>(rb, r, TOP, LE)];
  }
}

// Geometry of the whole-block VALU kernels: a block of 2^LB values is held by
// TB threads with E = 2^LE values each (contiguous runs: thread t holds
// positions t*E .. t*E+E-1); a workgroup of WG threads holds G blocks, each
// with its own lds_index-padded LDS copy for the group exchanges.
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
  // padded LDS index of position k * TB + t (coalesced order) and of t * E + r
  // (a thread's own run), written so that the compiler sees a per-thread base
  // plus a constant per k or r
  __device__ static int coal(int t, int k) {
    if constexpr (TB % 32 == 0) return t + (t >> 5) + k * (TB + TB / 32);
    else return lds_index(k * TB + t);
  }
  __device__ static int own(int t, int r) {
    if constexpr (E == 32) return t * 33 + r;
    else return lds_index(t * E + r);
  }
};

template <int LB>
__device__ __forceinline__ float inv_sqrt_block() {
  // 2^(-LB/2), exact for even LB
  return (LB & 1) ? 0.70710678118654752440f / (float)(1 << (LB >> 1)) : 1.0f / (float)(1 << (LB >> 1));
}

}  // namespace lwl
