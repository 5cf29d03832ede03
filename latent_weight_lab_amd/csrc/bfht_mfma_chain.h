// Matrix-core BlockFHT chain for block size 2^15 (gfx950, bf16 operands,
// float32 accumulation), shared by the generator kernels (bfht_mfma.hip) and
// the fused linear kernel (bfht_linear.hip).
//
// One workgroup of 8 waves (two per SIMD, so one wave's MFMAs overlap the
// other's VALU and LDS work) owns one 32768-element block; each lane holds 64
// values as 4 MFMA accumulator tiles of 16 floats.  The normalized Hadamard
// transform of a layer is split over three 5-bit groups of the position index
// (H_32768 = H_32 (x) H_32 (x) H_32), each applied as a 32x32 Walsh matrix
// with v_mfma_f32_32x32x16_bf16:
//
//   stage a, b: data is the A operand (rows = lanes 0-31, k = lane bit 5 and
//               4 register bits); the transformed group lands in lane bits
//               0-4 and the old lane bits move into the registers;
//   stage c:    data is the B operand; its 5 bits include all three wave
//               bits, so it follows one LDS exchange (64 KiB of bf16) that
//               swaps three already-transformed bits out to the wave index.
//
// Slot -> position bit assignment (p0..p14; Lk = lane bit k, Rk = bit k of the
// accumulator register index r = 0..15, Tk = bit k of the tile index,
// Wk = bit k of the wave index):
//
//   S0 (even layer start): L0-4 = p5-9, L5 = p10, R = p0 p1 p4 p11, T = p2 p3, W = p12 p13 p14
//   S1 (odd layer start):  L0-4 = p5-9, L5 = p12, R = p3 p2 p13 p14, T = p0 p1, W = p4 p10 p11
//
// An even layer starts in S0 and ends in S1, an odd one the reverse.  The sign
// layers meet the five bit-in-word bits (p0..p4) in registers, except p4 at
// S1, which is a wave bit; sign words (one 32-bit hash per 32 positions) are
// computed per lane and applied to packed bf16 pairs as XOR masks
// (word << (15 - b)) & 0x80008000, after a fixed permutation of the word's
// bits that puts the pair's two positions 16 bits apart (and a wave-uniform
// pre-shift for p4).
//
// Walsh entries are +-1/4, +-1/8, +-1/4 (exact in bf16); the remaining
// 2^(-L/2) of the L-layer normalization is folded into the last stage's
// entries, rounded to bf16 (relative error <= 2^-9).
//
// Reference semantics: latent_weight_lab/block_fht.py:84-109 (forward) and
// csrc/block_fht_ext_cuda.cu:185-223 (backward: the same chain with the sign
// layers in reverse order).
#pragma once

#include "bfht_device.h"
#include "bfht_launch.h"

namespace lwl {
namespace mfma15 {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kLog = 15;
constexpr int kB = 1 << kLog;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kTiles = 4;
constexpr int kChunks = kB / 8;  // 16-byte chunks of 8 bf16 in one block
// Exchange buffers: 4096 16-byte chunks of 8 bf16, stored by 8-byte halves in
// groups of 32 chunks: 256 bytes of the groups' low halves, then 256 bytes of
// their high halves (exchange_slot).  The 8-byte writes and reads of 32
// consecutive lanes then cover 256 consecutive LDS bytes (any gap between
// lanes costs LDS cycles in proportion), and the two halves of a chunk sit 256
// bytes apart, so one ds_read2_b64 fetches a whole MFMA operand into
// consecutive registers; two buffers back to back (128 KiB).
constexpr int kXBufBytes = kChunks * 16;
constexpr int kLdsBytes = 2 * kXBufBytes;
// Sign-word table after the exchange buffers: the words of sign layers 1..L
// (1024 per layer, 32 positions each), hashed once per block while the
// block's source loads are in flight.  A chain kernel's LDS is kChainLdsBytes.
constexpr int kMaxChainLayers = 3;
constexpr int kWordsPerLayer = kB / 32;
constexpr int kWordTableBytes = kMaxChainLayers * kWordsPerLayer * 4;
constexpr int kChainLdsBytes = kLdsBytes + kWordTableBytes;
constexpr uint32_t kPairSign = 0x80008000u;

__device__ __forceinline__ uint32_t pk(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Sign-word bit permutations exchanging bit-index bit 0 (resp. 3) with bit 4,
// so that the two positions of a packed pair sit 16 word bits apart.
__device__ __forceinline__ uint32_t swap_idx04(uint32_t x) {
  const uint32_t t = ((x >> 15) ^ x) & 0x0000aaaau;
  return x ^ t ^ (t << 15);
}
__device__ __forceinline__ uint32_t swap_idx34(uint32_t x) {
  const uint32_t t = ((x >> 8) ^ x) & 0x0000ff00u;
  return x ^ t ^ (t << 8);
}

// Walsh operands: for lane l and register pair (c, v), entries k = 16c +
// 8*(l>>5) + 2v + {0, 1}, o = l & 31, equal scale * (-1)^popcount(remap(k) & o)
// where remap moves k bit i to bit M[i].  The same registers serve as B operand
// (o = column) and as A operand (o = row).  make_walsh_table spells them out as
// bf16 pairs for the seven (permutation, scale) combinations the kernels use
// (walsh_words below builds the same words in registers, checked at compile time):
//   Q = (0,1,3,2,4) (k bits 2 and 3 exchanged), S = (1,0,2,3,4) (bits 0 and 1),
//   P = (0,2,1,3,4) (bits 1 and 2: the direct-store last layer, see run_chain);
//   bf16 0x3e80 = 1/4, 0x3e00 = 1/8, 0x3e35 = bf16(2^-2.5), 0x3db5 = bf16(2^-3.5).
enum { kWalshQ4, kWalshQ8, kWalshS4, kWalshSL1, kWalshSL3, kWalshPL1, kWalshPL3, kWalshSets };

struct WalshTable {
  uint32_t v[kWalshSets][64][8];
};

constexpr WalshTable make_walsh_table() {
  WalshTable tab{};
  const int perm[kWalshSets][5] = {{0, 1, 3, 2, 4}, {0, 1, 3, 2, 4}, {1, 0, 2, 3, 4}, {1, 0, 2, 3, 4},
                                   {1, 0, 2, 3, 4}, {0, 2, 1, 3, 4}, {0, 2, 1, 3, 4}};
  const uint32_t mag[kWalshSets] = {0x3e80u, 0x3e00u, 0x3e80u, 0x3e35u, 0x3db5u, 0x3e35u, 0x3db5u};
  for (int set = 0; set < kWalshSets; ++set)
    for (int lane = 0; lane < 64; ++lane)
      for (int c = 0; c < 2; ++c)
        for (int v = 0; v < 4; ++v) {
          uint32_t word = 0;
          for (int s = 0; s < 2; ++s) {
            const int k = 16 * c + 8 * (lane >> 5) + 2 * v + s;
            int km = 0;
            for (int i = 0; i < 5; ++i) km |= ((k >> i) & 1) << perm[set][i];
            int par = 0;
            for (int b = km & (lane & 31); b; b >>= 1) par ^= b & 1;
            word |= (mag[set] | (par ? 0x8000u : 0u)) << (16 * s);
          }
          tab.v[set][lane][4 * c + v] = word;
        }
  return tab;
}


// The same operands computed from the lane index (the table above is their
// definition; the chain builds them in registers, which saves every CU a
// 64 KiB read at the start of each block).  With o' the lane's column bits
// moved by the set's permutation (o'_i = bit perm[i] of o), entry k has the
// sign parity(k & o'), and k = 16c + 8h + 2v + s puts s, v0, v1, h, c at
// bits 0-4: word (c, v) = mag * 0x10001 with the high half's sign s-flipped by
// o'_0 and both signs flipped by h o'_3 ^ c o'_4 ^ v0 o'_1 ^ v1 o'_2.
__host__ __device__ constexpr uint32_t walsh_perm_bit(int set, int i) {
  // Q = (0,1,3,2,4) for the Q sets, S = (1,0,2,3,4) for the S sets, P = (0,2,1,3,4) for the P sets
  return (set == kWalshQ4 || set == kWalshQ8)     ? (i == 2 ? 3 : i == 3 ? 2 : i)
         : (set == kWalshPL1 || set == kWalshPL3) ? (i == 1 ? 2 : i == 2 ? 1 : i)
                                                  : (i == 0 ? 1 : i == 1 ? 0 : i);
}
__host__ __device__ constexpr uint32_t walsh_mag(int set) {
  return set == kWalshQ4 ? 0x3e80u : set == kWalshQ8 ? 0x3e00u : set == kWalshS4 ? 0x3e80u
       : (set == kWalshSL1 || set == kWalshPL1) ? 0x3e35u : 0x3db5u;
}
__host__ __device__ constexpr void walsh_words(int set, int lane, uint32_t (&w)[8]) {
  const uint32_t o = (uint32_t)lane & 31u, h = (uint32_t)lane >> 5;
  auto ob = [&](int i) { return (o >> walsh_perm_bit(set, i)) & 1u; };
  const uint32_t both = kPairSign;
  const uint32_t base = walsh_mag(set) * 0x10001u ^ (ob(0) << 31) ^ ((h & ob(3)) ? both : 0u);
  const uint32_t m1 = ob(1) ? both : 0u, m2 = ob(2) ? both : 0u, m4 = ob(4) ? both : 0u;
  w[0] = base;
  w[1] = base ^ m1;
  w[2] = base ^ m2;
  w[3] = w[1] ^ m2;
#pragma unroll
  for (int v = 0; v < 4; ++v) w[4 + v] = w[v] ^ m4;
}

// Compile-time check: the register construction equals the table, entry by entry.
constexpr bool walsh_words_match_table() {
  const WalshTable tab = make_walsh_table();
  for (int set = 0; set < kWalshSets; ++set)
    for (int lane = 0; lane < 64; ++lane) {
      uint32_t w[8] = {};
      walsh_words(set, lane, w);
      for (int i = 0; i < 8; ++i)
        if (w[i] != tab.v[set][lane][i]) return false;
    }
  return true;
}
static_assert(walsh_words_match_table(), "Walsh operands built in registers differ from their definition");

__device__ __forceinline__ void walsh_operand(int set, int lane, u32x4 (&h)[2]) {
  uint32_t w[8] = {};
  walsh_words(set, lane, w);
  h[0] = u32x4{w[0], w[1], w[2], w[3]};
  h[1] = u32x4{w[4], w[5], w[6], w[7]};
}

struct Ctx {
  int lane32, l5, wave;
  uint32_t bkey;
  uint32_t base0, base1;  // sign-word index bases in S0 and S1
  uint32_t gw0, gw1;      // 0xc2b2ae35 * (base + 1): the word term of the hash input
  int p4;                 // position bit p4 of this wave in S1
  int wid, rid;           // exchange slot bases (write / read side)
};

__device__ __forceinline__ Ctx make_ctx(uint32_t seed32, int64_t block) {
  Ctx x;
  const int tid = threadIdx.x;
  x.lane32 = tid & 31;
  x.l5 = (tid >> 5) & 1;
  x.wave = tid >> 6;
  x.bkey = block_key(seed32, block);
  // word = p >> 5.  S0 word bits: p5-9 = lane32, p10 = l5, p11 = slot, p12-14 = wave
  x.base0 = (uint32_t)(x.lane32 | (x.l5 << 5) | (x.wave << 7));
  // S1 word bits: p5-9 = lane32, p10-11 = wave >> 1, p12 = l5, p13-14 = slot
  x.base1 = (uint32_t)(x.lane32 | ((x.wave >> 1) << 5) | (x.l5 << 7));
  x.gw0 = 0xc2b2ae35u * (x.base0 + 1u);
  x.gw1 = 0xc2b2ae35u * (x.base1 + 1u);
  x.p4 = x.wave & 1;
  // exchange_slot of the chunk ids below, without their r / (t, c) terms
  x.wid = x.lane32 + ((x.wave & 1) << 5) + (x.l5 << 9) + ((x.wave >> 1) << 11);
  x.rid = x.lane32 + (x.wave << 8) + (x.l5 << 11);
  // Opaque to the compiler: knowing their range, it ORs a buffer's base (64
  // KiB) into every address instead of adding it once and folding the rest
  // into the LDS instructions' offset fields.
  asm("" : "+v"(x.wid), "+v"(x.rid));
  return x;
}

// Hash word of slot s: word index base + s * 2^shift (disjoint bits, so the
// word term 0xc2b2ae35 * (index + 1) is the lane's base term plus a constant).
__device__ __forceinline__ uint32_t slot_word(uint32_t key, uint32_t gw, int s, int shift) {
  return lowbias32(key ^ (gw + 0xc2b2ae35u * ((uint32_t)s << shift)));
}

// Sign words of one layer for this lane, inverted (set bit = flip) and
// permuted for the pair layout.  S0: 2 words, slot = p11.  S1: 4 words,
// slot = p13 + 2*p14, pre-shifted right by 8 when this wave's p4 is 1.

template <bool kOdd>
__device__ __forceinline__ void layer_words(const Ctx& x, int layer, uint32_t (&nw)[4]) {
  const uint32_t key = x.bkey ^ layer_key(layer);
#pragma unroll
  for (int s = 0; s < (kOdd ? 4 : 2); ++s) {
    const uint32_t w = ~(kOdd ? slot_word(key, x.gw1, s, 8) : slot_word(key, x.gw0, s, 6));
    nw[s] = kOdd ? (swap_idx34(w) >> (8 * x.p4)) : swap_idx04(w);
  }
  if (!kOdd) nw[2] = nw[3] = 0;
}

// Word pair {lo, hi} shifted left by s as one 64-bit value: one v_lshlrev_b64
// (full rate on gfx950, where LLVM would split a constant 64-bit shift into two
// 32-bit instructions).  The bits of lo shifted into hi land below bit s, and
// for s <= 15 below the pair-sign bits 15 and 31, so each dword of the result
// AND kPairSign is its own word's mask.
__device__ __forceinline__ u32x2 shl_pair(uint64_t pair, int s) {
  uint64_t r;
  asm("v_lshlrev_b64 %0, %1, %2" : "=v"(r) : "s"(s), "v"(pair));
  return u32x2{(uint32_t)r, (uint32_t)(r >> 32)};
}

// Sign masks of stage a's operands.  VGPR v of instruction c of tile t holds
// the packed pair j = (2v, 2v+1):
//   S0: j0 = p0 (pair), j1 = p1, j2 = p4, c = p11, t = (p2, p3)
//   S1: j0 = p3 (pair), j1 = p2, j2 = p13, c = p14, t = (p0, p1)
// and its XOR mask is (word << (15 - b)) & kPairSign with b the pair-layout bit
// of its low element: S0 word nw[c], b = (v >> 1) | (v & 1) << 1 | t << 2; S1
// word nw[(v >> 1) + 2c], b = t | (v & 1) << 2 (+ 8 p4, folded into the word).
// Instructions c = 0 and c = 1 of one VGPR share the shift, so one 64-bit shift
// of their two words gives both.  Pairs: S0 {nw[0], nw[1]}; S1 {nw[0], nw[2]}
// (v = 0, 1) and {nw[1], nw[3]} (v = 2, 3).
template <bool kOdd>
__device__ __forceinline__ void sign_pairs(const uint32_t (&nw)[4], uint64_t (&pairs)[2]) {
  if (kOdd) {
    pairs[0] = (uint64_t)nw[0] | ((uint64_t)nw[2] << 32);
    pairs[1] = (uint64_t)nw[1] | ((uint64_t)nw[3] << 32);
  } else {
    pairs[0] = pairs[1] = (uint64_t)nw[0] | ((uint64_t)nw[1] << 32);
  }
}
// a[c][v] ^= its mask, for both c, from the pairs above
template <bool kOdd>
__device__ __forceinline__ void sign_operands(u32x4 (&a)[2], const uint64_t (&pairs)[2], int t) {
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int b = kOdd ? (t | ((v & 1) << 2)) : ((v >> 1) | ((v & 1) << 1) | (t << 2));
    const u32x2 m = shl_pair(pairs[kOdd ? (v >> 1) : 0], 15 - b);
    a[0][v] ^= m[0] & kPairSign;
    a[1][v] ^= m[1] & kPairSign;
  }
}

__device__ __forceinline__ u32x4 pack8(const f32x16& a, int base) {
  u32x4 r;
  r[0] = pk(a[base + 0], a[base + 1]);
  r[1] = pk(a[base + 2], a[base + 3]);
  r[2] = pk(a[base + 4], a[base + 5]);
  r[3] = pk(a[base + 6], a[base + 7]);
  return r;
}

// Data as A operand: acc[t] <- packed(acc[t]) x H, sign layer fused when kSigned.
template <bool kSigned, bool kOdd>
__device__ __forceinline__ void stage_rows(f32x16 (&acc)[kTiles], const u32x4 (&h)[2],
                                           const uint32_t (&nw)[4]) {
  const f32x16 zero = {};
  uint64_t pairs[2];
  if (kSigned) sign_pairs<kOdd>(nw, pairs);
#pragma unroll
  for (int t = 0; t < kTiles; ++t) {
    u32x4 a[2] = {pack8(acc[t], 0), pack8(acc[t], 8)};
    if (kSigned) sign_operands<kOdd>(a, pairs, t);
    f32x16 d = mfma(a[0], h[0], zero);
    acc[t] = mfma(a[1], h[1], d);
  }
}

// Exchange: 16-byte chunk id (12 bits) of 8 packed values; each wave writes one
// 8-byte half (its 4 tiles at register r), the half being wave bit 0:
//   write: id = lane32 + (r&7)<<5 + l5<<8 + (r>>3)<<9 + (wave>>1)<<10, half = wave & 1
//   read:  id = lane32 + t<<5 + wave<<7 + l5<<10 + c<<11 (whole chunk = B operand)
// Half h of chunk id is 8-byte slot exchange_slot(id, h).
__host__ __device__ constexpr int exchange_slot(int id, int h) { return (id & 31) + (h << 5) + ((id >> 5) << 6); }

__device__ __forceinline__ void exchange_write(const f32x16 (&acc)[kTiles], u32x2* xbuf, const Ctx& x) {
  u32x2* half = xbuf + x.wid;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    u32x2 v;
    v[0] = pk(acc[0][r], acc[1][r]);
    v[1] = pk(acc[2][r], acc[3][r]);
    half[((r & 7) << 6) + ((r >> 3) << 10)] = v;
  }
}

__device__ __forceinline__ void exchange_read_stage_c(f32x16 (&acc)[kTiles], const u32x4 (&h)[2],
                                                      const u32x2* xbuf, int rid) {
  u32x4 b[kTiles][2];
  const u32x2* rd = xbuf + rid;
#pragma unroll
  for (int t = 0; t < kTiles; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int s = (t << 6) + (c << 12);
      const u32x2 lo = rd[s], hi = rd[s + 32];
      b[t][c] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  // All eight reads in flight before the first MFMA: left to itself the
  // compiler reuses one register set, and each read then waits out the LDS
  // latency alone.
  __builtin_amdgcn_sched_barrier(0);
  const f32x16 zero = {};
#pragma unroll
  for (int t = 0; t < kTiles; ++t) {
    f32x16 d = mfma(h[0], b[t][0], zero);
    acc[t] = mfma(h[1], b[t][1], d);
  }
}

// The slot bases above, checked against the chunk-id formulas.
constexpr bool exchange_slots_consistent() {
  for (int lane = 0; lane < 64; ++lane)
    for (int wave = 0; wave < kWaves; ++wave) {
      const int lane32 = lane & 31, l5 = lane >> 5;
      const int wid = lane32 + ((wave & 1) << 5) + (l5 << 9) + ((wave >> 1) << 11);
      const int rid = lane32 + (wave << 8) + (l5 << 11);
      for (int r = 0; r < 16; ++r) {
        const int id = lane32 + ((r & 7) << 5) + (l5 << 8) + ((r >> 3) << 9) + ((wave >> 1) << 10);
        if (wid + ((r & 7) << 6) + ((r >> 3) << 10) != exchange_slot(id, wave & 1)) return false;
      }
      for (int t = 0; t < kTiles; ++t)
        for (int c = 0; c < 2; ++c) {
          const int id = lane32 + (t << 5) + (wave << 7) + (l5 << 10) + (c << 11);
          const int s = rid + (t << 6) + (c << 12);
          if (s != exchange_slot(id, 0) || s + 32 != exchange_slot(id, 1)) return false;
        }
    }
  return true;
}
static_assert(exchange_slots_consistent(), "exchange slot bases disagree with the chunk layout");

// ---- direct-store last layer (odd L, whole blocks)
// The last exchange's read side is free (it goes through LDS), so the
// forward's last layer can end in a layout from which every lane stores whole
// 16-byte output chunks and each store instruction writes 1 KiB contiguous, with
// no LDS staging and no barrier after the chain:
//
//   F (end of the last layer): L0-4 = p4-8, L5 = p3, R = p2 p12 p13 p14, T = p0 p1, W = p9 p10 p11
//
// The writer is the regular one (S0, chunk id as exchange_write); the reader
// of lane (l32, l5) of wave w takes chunk id (l32 >> 1) | (w & 1) << 4 | t << 5 |
// (l32 & 1) << 7 | (w >> 1) << 8 | l5 << 10 | c << 11 (k bits p2, p3, p12, p13,
// p14 as before, columns p4-8 instead of p5-9), and stage c uses the Walsh set P,
// which sends k bits (p2, p3, p12, p13, p14) to row bits (r0, L5, r1, r2, r3).
// Lane (l32, l5) of wave w then holds output chunk k = (p12, p13, p14) = r >> 1
// of positions 8 l5 + 16 l32 + 512 w + 4096 k + 0..7, its 32-bit word q = (p1,
// p2) being the pair of tiles 2 (q & 1), 2 (q & 1) + 1 at register (q >> 1) |
// k << 1.  The LDS serves 128 bytes (32 banks of 4 bytes) per cycle, so an
// 8-byte access goes 16 lanes at a time, and each 16 lanes must fall on the 16
// 8-byte bank pairs (slot bits 0-3).  A write's 16 lanes differ in chunk-id
// bits 0-3, a read's in bits 0-2 and 7, so in this exchange the slot's bit 3 is
// chunk-id bit 3 XOR bit 7 (exchange_slot_final).
__host__ __device__ constexpr int exchange_slot_final(int id, int h) {
  return ((id & 23) | ((((id >> 3) ^ (id >> 7)) & 1) << 3)) + (h << 5) + ((id >> 5) << 6);
}

// exchange_write in exchange_slot_final: chunk-id bit 7 is register bit 2, so
// registers 4-7 and 12-15 write through the base with slot bit 3 flipped.
__device__ __forceinline__ void exchange_write_final(const f32x16 (&acc)[kTiles], u32x2* xbuf, const Ctx& x) {
  int w1 = x.wid ^ 8;
  asm("" : "+v"(w1));
  u32x2* half0 = xbuf + x.wid;
  u32x2* half1 = xbuf + w1;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    u32x2 v;
    v[0] = pk(acc[0][r], acc[1][r]);
    v[1] = pk(acc[2][r], acc[3][r]);
    ((r >> 2) & 1 ? half1 : half0)[((r & 7) << 6) + ((r >> 3) << 10)] = v;
  }
}

// Reader base slot of layout F (t << 6 and c << 12 added per operand).
__device__ __forceinline__ int rid_final(const Ctx& x) {
  int rid = ((x.lane32 >> 1) & 7) | ((((x.lane32 >> 4) ^ x.lane32) & 1) << 3) | ((x.wave & 1) << 4) |
            ((x.lane32 & 1) << 8) | ((x.wave >> 1) << 9) | (x.l5 << 11);
  asm("" : "+v"(rid));
  return rid;
}

constexpr bool exchange_final_consistent() {
  for (int lane = 0; lane < 64; ++lane)
    for (int wave = 0; wave < kWaves; ++wave) {
      const int l32 = lane & 31, l5 = lane >> 5;
      const int wid = l32 + ((wave & 1) << 5) + (l5 << 9) + ((wave >> 1) << 11);
      for (int r = 0; r < 16; ++r) {
        const int id = l32 + ((r & 7) << 5) + (l5 << 8) + ((r >> 3) << 9) + ((wave >> 1) << 10);
        if ((((r >> 2) & 1) ? wid ^ 8 : wid) + ((r & 7) << 6) + ((r >> 3) << 10) != exchange_slot_final(id, wave & 1))
          return false;
      }
      const int rid = ((l32 >> 1) & 7) | ((((l32 >> 4) ^ l32) & 1) << 3) | ((wave & 1) << 4) | ((l32 & 1) << 8) |
                      ((wave >> 1) << 9) | (l5 << 11);
      for (int t = 0; t < kTiles; ++t)
        for (int c = 0; c < 2; ++c) {
          const int id = (l32 >> 1) | ((wave & 1) << 4) | (t << 5) | ((l32 & 1) << 7) | ((wave >> 1) << 8) |
                         (l5 << 10) | (c << 11);
          const int s = rid + (t << 6) + (c << 12);
          if (s != exchange_slot_final(id, 0) || s + 32 != exchange_slot_final(id, 1)) return false;
        }
    }
  return true;
}
static_assert(exchange_final_consistent(), "final exchange slot bases disagree with the chunk layout");

// Even bit-in-word bits of x to the low half, odd ones to the high half, in
// order: bit j of the result is bit 2j of x, bit 16 + j is bit 2j + 1.
__host__ __device__ constexpr uint32_t unshuffle_bits(uint32_t x) {
  uint32_t t = (x ^ (x >> 1)) & 0x22222222u;
  x ^= t ^ (t << 1);
  t = (x ^ (x >> 2)) & 0x0c0c0c0cu;
  x ^= t ^ (t << 2);
  t = (x ^ (x >> 4)) & 0x00f000f0u;
  x ^= t ^ (t << 4);
  t = (x ^ (x >> 8)) & 0x0000ff00u;
  return x ^ t ^ (t << 8);
}
static_assert(unshuffle_bits(0x55555555u) == 0x0000ffffu && unshuffle_bits(0xaaaaaaaau) == 0xffff0000u &&
                  unshuffle_bits(0x00000006u) == 0x00010002u && unshuffle_bits(0x80000000u) == 0x80000000u,
              "unshuffle_bits");

// Fills the sign-word table (bytes kLdsBytes.. of the chain's LDS): slot j - 1
// holds the 1024 inverted words of sign layer sign_layer(j), j = 1..L, two per
// thread, in the form their reader applies: sign layer j < L is read by kernel
// layer j, whose stage a runs in S1 (j odd: bit permutation swap_idx34) or S0
// (j even: swap_idx04); the last one (j = L) is read by the output code, unpermuted.
// kDirect (the direct-store last layer): slot L - 1 holds the last layer's
// words as store_direct reads them, unshuffled (unshuffle_bits) and at index
// (w >> 7) + 8 (w & 127), so that the eight words of a lane's chunks k = w >> 7
// = 0..7 are consecutive.
template <int L, bool kDirect = false, class SignLayer>
__device__ __forceinline__ void fill_words(const Ctx& x, uint32_t* wtab, SignLayer sign_layer) {
  static_assert(L <= kMaxChainLayers, "word table holds kMaxChainLayers layers");
#pragma unroll
  for (int j = 1; j <= L; ++j) {
    const uint32_t key = x.bkey ^ layer_key(sign_layer(j));
#pragma unroll
    for (int h = 0; h < kWordsPerLayer / kThreads; ++h) {
      // consecutive threads write consecutive entries (a strided write would
      // serialize on the LDS banks); the direct slot's entry `at` holds word w
      const uint32_t at = (uint32_t)threadIdx.x + (uint32_t)(h * kThreads);
      const bool direct = kDirect && j == L;
      const uint32_t w = direct ? ((at & 7u) << 7) | (at >> 3) : at;
      uint32_t v = ~lowbias32(key ^ (0xc2b2ae35u * (w + 1u)));
      if (j < L)
        v = (j & 1) ? swap_idx34(v) : swap_idx04(v);
      else if (direct)
        v = unshuffle_bits(v);
      wtab[(j - 1) * kWordsPerLayer + at] = v;
    }
  }
}

// This lane's words of table slot `slot` as layer_words<kOdd> returns them
// (S1: slot = p13 + 2*p14, word index base1 + s*2^8; S0: slot = p11,
// base0 + s*2^6).  kPermuted: the slot holds the stage-a form (S1 words still
// take this wave's p4 pre-shift).
template <bool kOdd, bool kPermuted>
__device__ __forceinline__ void read_words(const Ctx& x, const uint32_t* wtab, int slot, uint32_t (&nw)[4]) {
  const uint32_t* t = wtab + slot * kWordsPerLayer;
  uint32_t base = kOdd ? x.base1 : x.base0;
  asm("" : "+v"(base));  // as the exchange bases: table offsets fold into the reads
#pragma unroll
  for (int s = 0; s < (kOdd ? 4 : 2); ++s) {
    const uint32_t v = t[base + (s << (kOdd ? 8 : 6))];
    nw[s] = (kOdd && kPermuted) ? (v >> (8 * x.p4)) : v;
  }
  if (!kOdd) nw[2] = nw[3] = 0;
}

// Runs the L-layer chain on a block whose unsigned input sits in `src`
// (src[t][c] = stage-a operand of tile t, instruction c, in S0; loads may still
// be in flight).  sign_layer(i) is the sign layer applied before kernel layer i
// (i < L) and after the last one (i = L); the latter's words are returned in
// `fin`.  On return acc holds the chain's result, before that last sign layer,
// in S1 (L odd) or S0 (L even).  Layer i exchanges through buffer i & 1 of
// `lds`: the previous readers of that buffer (layer i - 2) are past layer
// i - 1's barrier, and buffer L & 1 needs no barrier before its next writes.
// `lds` spans kChainLdsBytes; the sign words of layers 1..L are hashed into
// its table first (their loads' latency covers the hashing) and read after
// each layer's exchange barrier, which also orders the table's writes.
// kDirect (odd L): the last layer ends in layout F (see exchange_slot_final)
// instead of S1, and `fin` is not read (store_direct reads the last words).
template <int L, bool kDirect = false, class SignLayer>
__device__ __forceinline__ void run_chain(f32x16 (&acc)[kTiles], const Ctx& x, unsigned char* lds,
                                          const u32x4 (&src)[kTiles][2], SignLayer sign_layer,
                                          uint32_t (&fin)[4]) {
  static_assert(!kDirect || L % 2 == 1, "layout F follows an even layer's stages a, b");
  uint32_t* wtab = reinterpret_cast<uint32_t*>(lds + kLdsBytes);
  uint32_t nw[L][4];
  layer_words<false>(x, sign_layer(0), nw[0]);
  fill_words<L, kDirect>(x, wtab, sign_layer);
  const int lane = threadIdx.x & 63;
  // Stage a: Q/4 (even layers), S/4 (odd); stage b: Q/8; stage c: S/4 (even),
  // Q/4 (odd); the last stage c carries the residual 2^(-L/2): S/4*2^-0.5
  // (L = 1), Q/8 (L = 2), S/4*2^-1.5 (L = 3).
  u32x4 hq4[2], hq8[2], hs4[2], hlast[2];
  walsh_operand(kWalshQ4, lane, hq4);
  walsh_operand(kWalshQ8, lane, hq8);
  walsh_operand(kWalshS4, lane, hs4);
  walsh_operand(kDirect ? (L == 1 ? kWalshPL1 : kWalshPL3) : L == 1 ? kWalshSL1 : L == 2 ? kWalshQ8 : kWalshSL3, lane,
                hlast);
  const f32x16 zero = {};
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const bool odd = i & 1;
    const bool direct = kDirect && i == L - 1;
    if (i == 0) {
      uint64_t pairs[2];
      sign_pairs<false>(nw[0], pairs);
#pragma unroll
      for (int t = 0; t < kTiles; ++t) {
        u32x4 a[2] = {src[t][0], src[t][1]};
        sign_operands<false>(a, pairs, t);
        f32x16 d = mfma(a[0], hq4[0], zero);
        acc[t] = mfma(a[1], hq4[1], d);
      }
    } else if (odd) {
      stage_rows<true, true>(acc, hs4, nw[i]);
    } else {
      stage_rows<true, false>(acc, hq4, nw[i]);
    }
    stage_rows<false, false>(acc, hq8, nw[i]);
    u32x2* xbuf = reinterpret_cast<u32x2*>(lds + (i & 1) * kXBufBytes);
    if (direct)
      exchange_write_final(acc, xbuf, x);
    else
      exchange_write(acc, xbuf, x);
    __syncthreads();
    if (i + 1 < L) {
      if ((i + 1) & 1)
        read_words<true, true>(x, wtab, i, nw[i + 1]);
      else
        read_words<false, true>(x, wtab, i, nw[i + 1]);
    } else if (!kDirect) {
      read_words<(L % 2) == 1, false>(x, wtab, L - 1, fin);
    }
    exchange_read_stage_c(acc, i == L - 1 ? hlast : (odd ? hq4 : hs4), xbuf, direct ? rid_final(x) : x.rid);
  }
}

// Two blocks of the same latent through the chain together (the fused linear's
// two-block workgroups): the stages of both interleave, so one block's MFMAs
// and VALU work fill the other's dependency waits, and both share each
// layer's barrier and the source operands (the latent is the same; only the
// sign words differ).  LDS (kChain2LdsBytes): one exchange buffer per block
// (64 KiB each) and one sign-word table per block; a buffer is rewritten every
// layer, so layers after the first wait at a second barrier until every wave
// has read the previous layer's exchange.  Results as run_chain, per block.
constexpr int kChain2LdsBytes = 2 * kXBufBytes + 2 * kWordTableBytes;

template <int L, class SignLayer>
__device__ __forceinline__ void run_chain2(f32x16 (&acc)[2][kTiles], const Ctx (&x)[2], unsigned char* lds,
                                           const u32x4 (&src)[kTiles][2], SignLayer sign_layer,
                                           uint32_t (&fin)[2][4]) {
  uint32_t* wtab[2] = {reinterpret_cast<uint32_t*>(lds + 2 * kXBufBytes),
                       reinterpret_cast<uint32_t*>(lds + 2 * kXBufBytes + kWordTableBytes)};
  u32x2* xbuf[2] = {reinterpret_cast<u32x2*>(lds), reinterpret_cast<u32x2*>(lds + kXBufBytes)};
  uint32_t nw[2][L][4];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    layer_words<false>(x[b], sign_layer(0), nw[b][0]);
    fill_words<L>(x[b], wtab[b], sign_layer);
  }
  const int lane = threadIdx.x & 63;
  u32x4 hq4[2], hq8[2], hs4[2], hlast[2];
  walsh_operand(kWalshQ4, lane, hq4);
  walsh_operand(kWalshQ8, lane, hq8);
  walsh_operand(kWalshS4, lane, hs4);
  walsh_operand(L == 1 ? kWalshSL1 : L == 2 ? kWalshQ8 : kWalshSL3, lane, hlast);
  const f32x16 zero = {};
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const bool odd = i & 1;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      if (i == 0) {
        uint64_t pairs[2];
        sign_pairs<false>(nw[b][0], pairs);
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
          u32x4 a[2] = {src[t][0], src[t][1]};
          sign_operands<false>(a, pairs, t);
          f32x16 d = mfma(a[0], hq4[0], zero);
          acc[b][t] = mfma(a[1], hq4[1], d);
        }
      } else if (odd) {
        stage_rows<true, true>(acc[b], hs4, nw[b][i]);
      } else {
        stage_rows<true, false>(acc[b], hq4, nw[b][i]);
      }
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) stage_rows<false, false>(acc[b], hq8, nw[b][i]);
    if (i > 0) __syncthreads();  // every wave has read layer i - 1's exchange
#pragma unroll
    for (int b = 0; b < 2; ++b) exchange_write(acc[b], xbuf[b], x[b]);
    __syncthreads();
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      if (i + 1 < L) {
        if ((i + 1) & 1)
          read_words<true, true>(x[b], wtab[b], i, nw[b][i + 1]);
        else
          read_words<false, true>(x[b], wtab[b], i, nw[b][i + 1]);
      } else {
        read_words<(L % 2) == 1, false>(x[b], wtab[b], L - 1, fin[b]);
      }
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) exchange_read_stage_c(acc[b], i == L - 1 ? hlast : (odd ? hq4 : hs4), xbuf[b], x[b].rid);
  }
}

// Cache policy of the kernels' large output stores: sc0 | sc1 (system scope)
// writes through the XCD's L2.  The L2s of the XCDs are not coherent with each
// other, so a kernel's end writes every dirty L2 line back before the next
// kernel may read it; streaming the output through during the kernel instead
// removes that serial write-back from each launch (about 1 us for 16 MiB).
constexpr int kStreamStore = 1 | 16;

// Raw buffer resource over `bytes` bytes at `base`: loads past the end read 0,
// stores past the end are dropped (offsets are 32-bit).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Source operands in S0 from 16-byte chunks of 8 consecutive positions:
// chunk (t1, p4, c) holds p0..p2 for p3 = t1; its VGPR q (p1 = q&1, p2 = q>>1)
// is VGPR (q&1) + 2*p4 of operand (tile (q>>1) + 2*t1, instruction c).
// `load(p)` returns the 8 bf16 at block position p (a multiple of 8).
template <class Load>
__device__ __forceinline__ void load_source(const Ctx& x, Load load, u32x4 (&src)[kTiles][2]) {
  const int base = (x.lane32 << 5) + (x.l5 << 10) + (x.wave << 12);
#pragma unroll
  for (int t1 = 0; t1 < 2; ++t1)
#pragma unroll
    for (int p4 = 0; p4 < 2; ++p4)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const u32x4 v = load(base + ((t1 << 3) + (p4 << 4) + (c << 11)));
#pragma unroll
        for (int q = 0; q < 4; ++q) src[(q >> 1) + 2 * t1][c][(q & 1) + 2 * p4] = v[q];
      }
}

// Output chunk k = 0..7 of this lane (8 consecutive positions): its block
// position and its packed, signed content.
//   S1 (L odd):  r = (p3, p2, p13, p14), t = (p0, p1), wave = (p4, p10, p11), l5 = p12; k = (p3, p13, p14)
//   S0 (L even): r = (p0, p1, p4, p11), t = (p2, p3), wave = (p12, p13, p14), l5 = p10; k = (p3, p4, p11)
template <int L>
__device__ __forceinline__ int out_chunk_pos(const Ctx& x, int k) {
  if constexpr (L % 2 == 1)
    return ((k & 1) << 3) + (x.p4 << 4) + (x.lane32 << 5) + ((x.wave >> 1) << 10) + (x.l5 << 12) +
           ((k >> 1) << 13);
  else
    return ((k & 1) << 3) + (((k >> 1) & 1) << 4) + (x.lane32 << 5) + (x.l5 << 10) + ((k >> 2) << 11) +
           (x.wave << 12);
}

// All eight output chunks of this lane, packed and signed by the last sign layer.
//   S1: VGPR q of chunk k holds register r = (k & 1) | (q >> 1) << 1 | (k >> 1) << 2
//       of tiles 2 (q & 1) and 2 (q & 1) + 1 (p1 = q & 1, p2 = q >> 1, pair = p0);
//       word nw[k >> 1] (pair layout, pre-shifted by p4), bit b = 2 (q & 1) + 4 (q >> 1) + 8 (k & 1).
//   S0: VGPR q of chunk k holds registers r, r + 1 of tile (q >> 1) + 2 (k & 1),
//       r = 2 (q & 1) + 4 ((k >> 1) & 1) + 8 (k >> 2) (pair = p0); word nw[k >> 2],
//       bit b = ((k >> 1) & 1) + 2 (q & 1) + 4 (q >> 1) + 8 (k & 1).
// The masks come in pairs (shl_pair): in S1 chunks k and k + 2 (words k >> 1 and
// k >> 1 + 1), in S0 chunks k and k + 4 (words 0 and 1) share every shift.
template <int L>
__device__ __forceinline__ void out_chunks(const f32x16 (&acc)[kTiles], const uint32_t (&nw)[4], const Ctx& x,
                                           u32x4 (&v)[8]) {
  if constexpr (L % 2 == 1) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = swap_idx04(nw[j]) >> x.p4;
    const uint64_t pair[2] = {(uint64_t)w[0] | ((uint64_t)w[1] << 32), (uint64_t)w[2] | ((uint64_t)w[3] << 32)};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int r0 = (k & 1) | ((k >> 1) << 2);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = r0 | ((q >> 1) << 1);
        v[k][q] = pk(acc[2 * (q & 1)][r], acc[2 * (q & 1) + 1][r]);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if ((k >> 1) & 1) continue;  // chunk k + 2 takes the pair's high word
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int b = ((q & 1) << 1) | ((q >> 1) << 2) | ((k & 1) << 3);
        const u32x2 m = shl_pair(pair[k >> 2], 15 - b);
        v[k][q] ^= m[0] & kPairSign;
        v[k + 2][q] ^= m[1] & kPairSign;
      }
    }
  } else {
    const uint64_t pair = (uint64_t)swap_idx04(nw[0]) | ((uint64_t)swap_idx04(nw[1]) << 32);
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t = (q >> 1) + 2 * (k & 1);
        const int r = 2 * (q & 1) + 4 * ((k >> 1) & 1) + 8 * (k >> 2);
        v[k][q] = pk(acc[t][r], acc[t][r + 1]);
      }
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int b = ((k >> 1) & 1) | ((q & 1) << 1) | ((q >> 1) << 2) | ((k & 1) << 3);
        const u32x2 m = shl_pair(pair, 15 - b);
        v[k][q] ^= m[0] & kPairSign;
        v[k + 4][q] ^= m[1] & kPairSign;
      }
  }
}

// Slot of 16-byte output chunk c in the staging buffer.  The lanes of one
// staging write hold chunks 4 apart (c = 4 * lane32 + const); XOR-ing bits
// 3-4 into bits 0-1 spreads any 8 consecutive lanes over the 8 16-byte bank
// groups of a 128-byte LDS row, and every aligned group of 8 chunks stays in
// place as a whole, so reads of consecutive chunks are conflict-free too.
__device__ __forceinline__ int stage_slot(int c) { return c ^ ((c >> 3) & 3); }

// Stages the chain's result (acc, before the last sign layer, words `nw`) as
// signed bf16 in block-position order into `stage` (4096 16-byte chunks at
// stage_slot(c)).  The caller synchronizes before reading.
template <int L>
__device__ __forceinline__ void stage_output(const f32x16 (&acc)[kTiles], const uint32_t (&nw)[4], const Ctx& x,
                                             u32x4* stage) {
  u32x4 v[8];
  out_chunks<L>(acc, nw, x, v);
#pragma unroll
  for (int k = 0; k < 8; ++k) stage[stage_slot(out_chunk_pos<L>(x, k) >> 3)] = v[k];
}

// The 8 bf16 of a chunk times `scale`, rounded to bf16 (torch's bf16 * scalar).
__device__ __forceinline__ u32x4 scale_chunk(u32x4 v, float scale) {
#pragma unroll
  for (int k = 0; k < 4; ++k)
    v[k] = pk(__uint_as_float(v[k] << 16) * scale, __uint_as_float(v[k] & 0xffff0000u) * scale);
  return v;
}

// The forward's whole block from layout F (run_chain<L, true>): the last sign
// layer and 16-byte write-through stores of whole chunks, 1 KiB contiguous per
// instruction, straight from registers.  `words` is the table slot the chain
// filled for it (fill_words<L, true>): a lane's eight words, those of its chunks
// k = 0..7, are consecutive; the chunk's bit-in-word bits are p0-p2 (in the
// chunk) + 8 p3 (l5) + 16 p4 (l32 bit 0), so after the shift by 4 (l5 + 2 p4) of
// the unshuffled word, bit q (bit 16 + q) holds the sign of the chunk's value 2q
// (2q + 1), the pair of word q, and (w << (15 - q)) & kPairSign is its mask.
// Each value is multiplied by `scale` (exact when 1) after its rounding to bf16.
__device__ __forceinline__ void store_direct(const f32x16 (&acc)[kTiles], const Ctx& x, const uint32_t* words,
                                             __amdgpu_buffer_rsrc_t out_r, float scale = 1.0f) {
  const u32x4* wt = reinterpret_cast<const u32x4*>(words) + 2 * ((x.lane32 >> 1) + 16 * x.wave);
  const u32x4 wa = wt[0], wb = wt[1];
  const int sh = 4 * (x.l5 + 2 * (x.lane32 & 1));
  const uint32_t w[8] = {wa[0] >> sh, wa[1] >> sh, wa[2] >> sh, wa[3] >> sh,
                         wb[0] >> sh, wb[1] >> sh, wb[2] >> sh, wb[3] >> sh};
  u32x4 v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = (q >> 1) | (k << 1);
      v[k][q] = pk(acc[2 * (q & 1)][r], acc[2 * (q & 1) + 1][r]);
    }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint64_t pair = (uint64_t)w[k] | ((uint64_t)w[k + 4] << 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x2 m = shl_pair(pair, 15 - q);
      v[k][q] ^= m[0] & kPairSign;
      v[k + 4][q] ^= m[1] & kPairSign;
    }
  }
  if (scale != 1.0f) {
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = scale_chunk(v[k], scale);
  }
  const int base = 16 * x.l5 + 32 * x.lane32 + 1024 * x.wave;
#pragma unroll
  for (int k = 0; k < 8; ++k) __builtin_amdgcn_raw_buffer_store_b128(v[k], out_r, base + 8192 * k, 0, kStreamStore);
}

// Slot of 4-float chunk c in write_partial_row's staging.  A ds_write_b128
// serves 8 consecutive lanes per LDS cycle over 32 banks, a ds_read_b128 16
// lanes over 64 banks: lanes 0-3, 12-15, 20-23, 24-27 together and lanes 4-7,
// 8-11, 16-19, 28-31 together (the same for 32-63; measured with two active
// lanes at a time).  The writes hold chunks 8 apart (chunk bits 3-5 vary over
// 8 lanes), so bits 3-5 are XORed into bits 0-2 as a permutation; bit 4 going
// to bit 0 also sets the bf16 reads' pairs of chunks 2 (base + lane) + {0, 1}
// of each cycle's four lane quads apart (with bits 3-5 in place, two of the
// quads shared the 16-byte bank groups).
__device__ __forceinline__ int prow_slot(int c) {
  return c ^ ((c >> 4) & 1) ^ (((c >> 3) & 1) << 1) ^ (((c >> 5) & 1) << 2);
}

// Backward tail: applies D_0 (inverted words `nw` of the chain's last sign
// layer, in the chain's output layout) to the adjoint chain's result and
// writes scale * the float32 row of the first n block positions to prow,
// staged through the exchange space (128 KiB; 4-float chunk c at prow_slot(c)).
// kExact: n % 4 == 0 (whole 16-byte stores; stores past n are dropped).
template <int L, bool kExact, class P = float>
__device__ __forceinline__ void write_partial_row(const f32x16 (&acc)[kTiles], const uint32_t (&nw)[4],
                                                  const Ctx& x, unsigned char* lds, P* prow, int n,
                                                  float scale) {
  auto flip = [](float v, uint32_t w, int b) {
    return __uint_as_float(__float_as_uint(v) ^ ((w << (31 - b)) & 0x80000000u));
  };
  f32x4* stage = reinterpret_cast<f32x4*>(lds);  // all 128 KiB
  // bf16 rows of odd L go out in two halves: register r holds position bit 14
  // = r >> 3, so the first half's stores leave while the second half is staged.
  constexpr int kPhases = (L % 2 == 1 && sizeof(P) == 2) ? 2 : 1;
  __syncthreads();  // every wave has read its last exchange
  const auto p_r = rsrc(prow, (uint32_t)n * (uint32_t)sizeof(P));
#pragma unroll
  for (int ph = 0; ph < kPhases; ++ph) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (kPhases > 1 && (r >> 3) != ph) continue;
      f32x4 v;
      int p;
      if constexpr (L % 2 == 1) {
        // S1: chunk = the 4 tiles at register r (p0, p1 = tile bits)
        p = (((r >> 1) & 1) << 2) + ((r & 1) << 3) + (x.p4 << 4) + (x.lane32 << 5) + ((x.wave >> 1) << 10) +
            (x.l5 << 12) + ((r >> 2) << 13);
        const uint32_t w = nw[r >> 2];
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = scale * flip(acc[t][r], w, (p & 31) + t);
      } else {
        // S0: chunk = registers r0 .. r0+3 of tile t (p0, p1 = register bits)
        const int t = r & 3, r0 = (r >> 2) << 2;
        p = (t << 2) + (((r0 >> 2) & 1) << 4) + (x.lane32 << 5) + (x.l5 << 10) + ((r0 >> 3) << 11) +
            (x.wave << 12);
        const uint32_t w = nw[r0 >> 3];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = scale * flip(acc[t][r0 + e], w, (p & 31) + e);
      }
      const int c = p >> 2;
      stage[prow_slot(c)] = v;
    }
    __syncthreads();
    if constexpr (sizeof(P) == 4) {
#pragma unroll
      for (int i = 0; i < (kB / 4) / kThreads; ++i) {
        const int c = i * kThreads + (int)threadIdx.x;
        const f32x4 v = stage[prow_slot(c)];
        const int p = c * 4;
        if (kExact || p + 4 <= n) {
          __builtin_amdgcn_raw_buffer_store_b128(v, p_r, p * 4, 0, kStreamStore);  // dropped past n
        } else if (p < n) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (p + e < n) prow[p + e] = v[e];
        }
      }
    } else {  // bf16 row: two staged chunks (8 positions) per 16-byte store
      constexpr int kPer = (kB / 8) / kPhases;
#pragma unroll
      for (int i = 0; i < kPer / kThreads; ++i) {
        const int c2 = ph * kPer + i * kThreads + (int)threadIdx.x;
        const f32x4 a = stage[prow_slot(2 * c2)];
        const f32x4 b = stage[prow_slot(2 * c2 + 1)];
        const u32x4 v = {pk(a[0], a[1]), pk(a[2], a[3]), pk(b[0], b[1]), pk(b[2], b[3])};
        const int p = c2 * 8;
        if (kExact || p + 8 <= n) {
          __builtin_amdgcn_raw_buffer_store_b128(v, p_r, p * 2, 0, kStreamStore);  // dropped past n
        } else if (p < n) {
          uint16_t* row16 = reinterpret_cast<uint16_t*>(prow);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (p + e < n) row16[p + e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
  }
}

// Loads the S0 source operands of a block from the latent (n bf16 elements,
// zero past the end).  kExact: n % 8 == 0, so no 16-byte chunk straddles the end.
template <bool kExact = false>
__device__ __forceinline__ void load_latent(const Ctx& x, const __bf16* latent, int n, u32x4 (&src)[kTiles][2]) {
  const auto lat_r = rsrc(latent, (uint32_t)n * 2u);
  const uint16_t* lat16 = reinterpret_cast<const uint16_t*>(latent);
  const bool tail = !kExact && (n & 7) != 0;
  load_source(
      x,
      [&](int p) -> u32x4 {
        // sc0: every CU reads each latent line once, from its XCD's L2 (config 2:
        // within run-to-run spread of the default policy, 8.86-9.02 us; sc1 or nt,
        // which miss the L2, take ~9.9 us)
        u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(lat_r, p * 2, 0, 1);  // 0 past n
        if (tail && p < n && p + 8 > n) {  // straddles the end of the latent: exact element loads
          v = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (p + e < n) v[e >> 1] |= (uint32_t)lat16[p + e] << (16 * (e & 1));
        }
        return v;
      },
      src);
}

}  // namespace mfma15
}  // namespace lwl
