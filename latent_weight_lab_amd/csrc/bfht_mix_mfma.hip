// Signed activation FHT on the matrix cores: float16 / bfloat16 rows of P =
// 1024 or 4096 values (GPT-2's 768 and 3072 features, padded).
//
// y = (S H S pad(x))[:F] per row (reference examples/nanogpt/model.py:180-218:
// pad to P, multiply by the ±1 sign buffer, normalized_fht_last_dim, multiply
// by the signs again, keep the first F), as two radix-32 stages on
// v_mfma_f32_32x32x16_{bf16,f16} with float32 accumulation and, at P = 4096, a
// radix-4 stage in float32 registers.  The input is already in the I/O type, so
// the first stage's operands are exact; the second stage's operands are the
// first stage's float32 results rounded once to the I/O type, and the output
// is rounded once more (the reference's torch loop rounds to the activation
// type after each of its log2 P stages).
//
// A wave holds 4 tiles of 1024 values (64 lanes x 16 accumulator registers):
// the 4 quarters of one row at P = 4096, four rows at P = 1024.  Position bits
// of a tile (p0..p9; at P = 4096 the tile index is p10, p11):
//   load, the stage-1 A operand of instruction c: lanes 0-31 = p3..p7, lane bit
//        5 = p8, c = p9, the 8 values of the 16-byte operand = p0..p2, so one
//        load instruction reads 1 KiB contiguous;
//   stage 1 transforms (p0, p1, p2, p8, p9) with the Walsh matrix's k bits 2
//        and 3 exchanged (p8 lands on output column bit 2, p2 on bit 3); after
//        it lanes 0-31 = (p0, p1, p8, p2, p9) and accumulator register 4i + j
//        holds j0 = p3, j1 = p4, i0 = p6, i1 = p7, lane bit 5 = p5;
//   stage 2 transforms (p3, p4, p6, p5, p7): each 8-register half of the
//        accumulators is one A operand (c = i1); after it lanes 0-31 = (p3,
//        p4, p6, p5, p7), lane bit 5 = p8 and register 4i + j holds j0 = p0,
//        j1 = p1, i0 = p2, i1 = p9, so registers 8 i1 .. 8 i1 + 7 are 8
//        consecutive positions and one 16-byte store instruction writes 1 KiB
//        contiguous.
// Output rows of 32x32x16: register 4i + j of lane l is row 8i + 4 (l >> 5) + j,
// column l & 31; A operand: lane l holds row l & 31, k = 8 (l >> 5) .. + 7.
#include "bfht_block.h"

namespace lwl {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kMixMfmaWaves = 4;        // waves per workgroup
// workgroups (each wave loops over its row groups): 4 per CU at P = 1024, one
// per CU (one wave per SIMD) at P = 4096, which streams faster than two per CU
// (8192 x 3072 bf16: 17.9 us against 21.0 us; 32768 x 3072: 64 against 84 us)
constexpr int64_t kMixMfmaMaxGrid[2] = {1024, 256};
// Cache policy of the row loads: nt (each row is read once; with the default
// policy the same kernel streams at ~80 % of this rate)
constexpr int kMixStreamLoad = 2;
// Output stores write through the XCD's L2 (sc0 sc1): a kernel's end writes every
// dirty L2 line back, which for tens of MB of output is a serial tail.
constexpr int kMixStreamStore = 1 | 16;

// Walsh B operands of the two stages: lane l, instruction c, register v holds
// the pair k = 16c + 8 (l >> 5) + 2v + {0, 1} of column n = l & 31, entry
// mag * (-1)^popcount(pi(k) & n), pi = exchange of k bits 2 and 3 in stage 1
// and the identity in stage 2.  mag: stage 1 1/4, stage 2 1/8 (P = 1024) or
// 1/16 (P = 4096, whose radix-4 stage adds unscaled), so the product is
// 1/sqrt(P), every entry exact in both types.
struct MixWalsh {
  uint32_t w[2][64][8];
};

constexpr int mix_walsh_k(int stage, int k) {
  return stage == 0 ? ((k & 0x13) | ((k >> 1) & 4) | ((k << 1) & 8)) : k;
}

constexpr MixWalsh make_mix_walsh(uint32_t mag1, uint32_t mag2) {
  MixWalsh t{};
  for (int s = 0; s < 2; ++s)
    for (int lane = 0; lane < 64; ++lane)
      for (int c = 0; c < 2; ++c)
        for (int v = 0; v < 4; ++v) {
          uint32_t word = 0;
          for (int h = 0; h < 2; ++h) {
            const int k = mix_walsh_k(s, 16 * c + 8 * (lane >> 5) + 2 * v + h);
            int par = 0;
            for (int b = k & (lane & 31); b; b >>= 1) par ^= b & 1;
            word |= ((s == 0 ? mag1 : mag2) | (par ? 0x8000u : 0u)) << (16 * h);
          }
          t.w[s][lane][4 * c + v] = word;
        }
  return t;
}

// Check: each stage's 32 x 32 matrix (entries read back from the words) has
// orthogonal columns of equal norm, i.e. it is a scaled Hadamard matrix, and
// stage 2 is the Sylvester matrix itself (entry (k, n) sign = parity(k & n)).
constexpr bool mix_walsh_valid(const MixWalsh& t) {
  auto sign = [&](int s, int k, int n) {
    // k -> (c, lane half, v, h); any lane with column n and that half holds it
    const int c = k >> 4, half = (k >> 3) & 1, v = (k >> 1) & 3, h = k & 1;
    const uint32_t word = t.w[s][n + 32 * half][4 * c + v];
    return ((word >> (16 * h + 15)) & 1u) ? -1 : 1;
  };
  for (int s = 0; s < 2; ++s)
    for (int n = 0; n < 32; ++n)
      for (int m = 0; m < 32; ++m) {
        int dot = 0;
        for (int k = 0; k < 32; ++k) dot += sign(s, k, n) * sign(s, k, m);
        if (dot != (n == m ? 32 : 0)) return false;
      }
  for (int k = 0; k < 32; ++k)
    for (int n = 0; n < 32; ++n) {
      int par = 0;
      for (int b = k & n; b; b >>= 1) par ^= b & 1;
      if (sign(1, k, n) != (par ? -1 : 1)) return false;
    }
  return true;
}

// bf16 1/4, 1/8, 1/16 = 0x3e80, 0x3e00, 0x3d80; f16 = 0x3400, 0x3000, 0x2c00
__constant__ constexpr MixWalsh kMixWalshBf16_10 = make_mix_walsh(0x3e80u, 0x3e00u);
__constant__ constexpr MixWalsh kMixWalshBf16_12 = make_mix_walsh(0x3e80u, 0x3d80u);
__constant__ constexpr MixWalsh kMixWalshF16_10 = make_mix_walsh(0x3400u, 0x3000u);
__constant__ constexpr MixWalsh kMixWalshF16_12 = make_mix_walsh(0x3400u, 0x2c00u);
static_assert(mix_walsh_valid(make_mix_walsh(0x3e80u, 0x3d80u)), "stage matrices are not Hadamard");

template <class T>
struct MixMfmaType;
template <>
struct MixMfmaType<bf16> {
  __device__ static f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  __device__ static uint32_t pk(float lo, float hi) {
    const f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  }
  template <int LB>
  __device__ static const MixWalsh& walsh() {
    return LB == 12 ? kMixWalshBf16_12 : kMixWalshBf16_10;
  }
};
template <>
struct MixMfmaType<f16> {
  __device__ static f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  __device__ static uint32_t pk(float lo, float hi) {
    const f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  }
  template <int LB>
  __device__ static const MixWalsh& walsh() {
    return LB == 12 ? kMixWalshF16_12 : kMixWalshF16_10;
  }
};

// Sign bits of the pair at positions p, p + 1 in the packed layout (bit 15 of
// the low half, bit 31 of the high half).
__device__ __forceinline__ uint32_t pair_mask(const float* sgn, int p) {
  return (sgn[p] < 0.0f ? 0x8000u : 0u) | (sgn[p + 1] < 0.0f ? 0x80000000u : 0u);
}

// kVec: x and out start on the 16-byte grid and the rows hold whole 16-byte
// chunks (features % 8 == 0), so a chunk is one 16-byte access; otherwise the
// chunks are read and written element by element (the same arithmetic).
//
// Each wave loops over its row groups with the next group's loads in flight
// while it transforms the current one (two register sets, used in turn).  The
// sign masks (per lane: 8 in-operand and 8 out-chunk words of four packed
// pairs each) are the same in every wave: at P = 4096 they sit in LDS, built
// once per workgroup and read per row group (registers hold the two row
// groups instead); at P = 1024 the 16 words stay in registers.
template <int LB, class T, bool kVec>
__global__ __launch_bounds__(64 * kMixMfmaWaves) __attribute__((amdgpu_waves_per_eu(kVec && LB == 10 ? 4 : 2))) void bfht_mix_mfma(const T* x, T* out,
                                                                   const float* __restrict__ signs, int64_t rows,
                                                                   int features) {
  static_assert(LB == 10 || LB == 12, "rows of 1024 or 4096 values");
  using Ty = MixMfmaType<T>;
  constexpr int P = 1 << LB;
  constexpr bool kQuarters = LB == 12;  // the tiles are the quarters of one row
  constexpr int kRowsPerWave = kQuarters ? 1 : 4;
  constexpr int kThreads = 64 * kMixMfmaWaves;
  __shared__ float sgn[P];
  // P = 4096: mask group j (0..7 input chunk (t, c) = j; 8..15 output chunk (t, i1) = j - 8) of lane l
  // at mtab[j * 64 + l] (consecutive lanes on consecutive 16-byte slots: conflict-free reads)
  __shared__ u32x4 mtab[kQuarters ? 16 * 64 : 1];
  const int lane = threadIdx.x & 63, l32 = lane & 31, l5 = lane >> 5;
  // first position of this lane's input chunk (+ 512 c + 1024 t) and output chunk (+ 512 i1 + 1024 t)
  const int pin = 8 * l32 + 256 * l5;
  const int pout = 8 * (l32 & 1) + 16 * ((l32 >> 1) & 1) + 64 * ((l32 >> 2) & 1) + 32 * ((l32 >> 3) & 1) +
                   128 * (l32 >> 4) + 256 * l5;
  const int64_t groups = (rows + kRowsPerWave - 1) / kRowsPerWave;
  const int64_t nwaves = (int64_t)gridDim.x * kMixMfmaWaves;
  const int64_t wave = (int64_t)blockIdx.x * kMixMfmaWaves + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const uint32_t row_bytes = (uint32_t)features * (uint32_t)sizeof(T);
  auto tile_row = [](int t) { return kQuarters ? 0 : t; };
  auto tile_base = [](int t) { return kQuarters ? 1024 * t : 0; };
  // buffer of row q of group g (rows past the end: empty, reads 0, writes dropped)
  auto row_rsrc = [&](const T* base, int64_t g, int q) {
    const int64_t row = g * kRowsPerWave + q;
    const bool ok = row < rows;
    return tile_rsrc(base + (ok ? row : 0) * features, ok ? row_bytes : 0u);
  };

  auto load_group = [&](int64_t g, u32x4 (&a)[4][2]) {
    __amdgpu_buffer_rsrc_t xr[kRowsPerWave];
#pragma unroll
    for (int q = 0; q < kRowsPerWave; ++q) xr[q] = row_rsrc(x, g, q);
    if constexpr (kVec) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          a[t][c] = __builtin_amdgcn_raw_buffer_load_b128(
              xr[tile_row(t)], (int)((uint32_t)(pin + 512 * c + tile_base(t)) * sizeof(T)), 0, kMixStreamLoad);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int p = pin + 512 * c + tile_base(t);
          u32x4 v = {0u, 0u, 0u, 0u};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(xr[tile_row(t)], (int)((uint32_t)(p + e) * 2u), 0, 0);
            v[e >> 1] |= h << (16 * (e & 1));
          }
          a[t][c] = v;
        }
    }
  };

  // This thread's share of the sign table and the first row group's loads go
  // out together, the table's first (a wave past the last group reads empty
  // rows, so the group's loads need no branch).  The table's writes then wait
  // for the sign loads alone (the wait counter retires loads in order), and the
  // group's loads stay in flight while the masks are built; a loop of one load
  // and one wait per iteration waited out a memory round trip per iteration
  // before the first product (rows of 768: 5.23 -> 4.57 us).  The Walsh
  // operands, from constant memory, are loaded where first used, behind the
  // masks' LDS reads (loaded up front they measured no faster).
  static_assert(P % kThreads == 0, "the sign table in whole rounds of the workgroup");
  constexpr int kSgnPer = P / kThreads;
  float sv[kSgnPer];
#pragma unroll
  for (int j = 0; j < kSgnPer; ++j) sv[j] = signs[threadIdx.x + j * kThreads];
  const MixWalsh& W = Ty::template walsh<LB>();
  u32x4 h1[2], h2[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    h1[c] = *reinterpret_cast<const u32x4*>(&W.w[0][lane][4 * c]);
    h2[c] = *reinterpret_cast<const u32x4*>(&W.w[1][lane][4 * c]);
  }
  u32x4 cur[4][2];
  load_group(wave < groups ? wave : groups, cur);

#pragma unroll
  for (int j = 0; j < kSgnPer; ++j) sgn[threadIdx.x + j * kThreads] = sv[j];
  __syncthreads();

  auto mask4 = [&](int p) {
    u32x4 m;
#pragma unroll
    for (int v = 0; v < 4; ++v) m[v] = pair_mask(sgn, p + 2 * v);
    return m;
  };
  u32x4 m_in[2], m_out[2];  // P = 1024: one set for all four rows
  if constexpr (kQuarters) {
    const int w = threadIdx.x >> 6;  // wave w builds groups 4w .. 4w + 3 of its lane
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = 4 * w + q, t = (j & 7) >> 1, c = j & 1;
      mtab[j * 64 + lane] = mask4((j < 8 ? pin : pout) + 512 * c + 1024 * t);
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      m_in[c] = mask4(pin + 512 * c);
      m_out[c] = mask4(pout + 512 * c);
    }
  }
  const f32x16 zero = {};
  auto transform_store = [&](int64_t g, const u32x4 (&a)[4][2]) {
    // the mask table's lane index, opaque per row group: the 16 mask reads stay
    // in the loop instead of being held in 64 registers across it
    int ml = lane;
    asm volatile("" : "+v"(ml));
    // stage 1: signs, then (p0, p1, p2, p8, p9)
    f32x16 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const u32x4 mi0 = kQuarters ? mtab[(2 * t) * 64 + ml] : m_in[0];
      const u32x4 mi1 = kQuarters ? mtab[(2 * t + 1) * 64 + ml] : m_in[1];
      acc[t] = Ty::mfma(a[t][0] ^ mi0, h1[0], zero);
      acc[t] = Ty::mfma(a[t][1] ^ mi1, h1[1], acc[t]);
    }
    // stage 2: (p3, p4, p6, p5, p7), operands rounded to the I/O type
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      u32x4 b0, b1;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        b0[q] = Ty::pk(acc[t][2 * q], acc[t][2 * q + 1]);
        b1[q] = Ty::pk(acc[t][8 + 2 * q], acc[t][8 + 2 * q + 1]);
      }
      acc[t] = Ty::mfma(b0, h2[0], zero);
      acc[t] = Ty::mfma(b1, h2[1], acc[t]);
    }
    if constexpr (kQuarters) {  // stage 3: (p10, p11) across the tiles, unscaled
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float b0 = acc[0][r] + acc[1][r], b1 = acc[0][r] - acc[1][r];
        const float b2 = acc[2][r] + acc[3][r], b3 = acc[2][r] - acc[3][r];
        acc[0][r] = b0 + b2;
        acc[1][r] = b1 + b3;
        acc[2][r] = b0 - b2;
        acc[3][r] = b1 - b3;
      }
    }
    // output: chunk (t, i1) = registers 8 i1 .. 8 i1 + 7 of tile t, signed
    __amdgpu_buffer_rsrc_t orr[kRowsPerWave];
#pragma unroll
    for (int q = 0; q < kRowsPerWave; ++q) orr[q] = row_rsrc(out, g, q);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i1 = 0; i1 < 2; ++i1) {
        const u32x4 mo = kQuarters ? mtab[(8 + 2 * t + i1) * 64 + ml] : m_out[i1];
        u32x4 w;
#pragma unroll
        for (int q = 0; q < 4; ++q) w[q] = Ty::pk(acc[t][8 * i1 + 2 * q], acc[t][8 * i1 + 2 * q + 1]) ^ mo[q];
        const int p = pout + 512 * i1 + tile_base(t);
        if constexpr (kVec) {
          __builtin_amdgcn_raw_buffer_store_b128(w, orr[tile_row(t)], (int)((uint32_t)p * sizeof(T)), 0,
                                                 kMixStreamStore);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(w[e >> 1] >> (16 * (e & 1))), orr[tile_row(t)],
                                                  (int)((uint32_t)(p + e) * 2u), 0, kMixStreamStore);
        }
      }
  };

  // row groups g, g + nwaves, ...: the next group's loads are issued before
  // the current group is transformed (past the last group they read nothing).
  // A group's stores follow all of its loads, so out may alias x.
  for (int64_t g = wave; g < groups; g += nwaves) {
    u32x4 nxt[4][2];
    load_group(g + nwaves, nxt);
    transform_store(g, cur);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) cur[t][c] = nxt[t][c];
  }
}

template <int LB, class T>
hipError_t launch_mix_mfma_lb(const void* x, void* out, const float* signs, int64_t rows, int64_t features,
                              hipStream_t s) {
  constexpr int kRowsPerWave = LB == 12 ? 1 : 4;
  const int64_t groups = (rows + kRowsPerWave - 1) / kRowsPerWave;
  const int64_t wgs = (groups + kMixMfmaWaves - 1) / kMixMfmaWaves;
  const int64_t most = kMixMfmaMaxGrid[LB == 12];
  const int64_t grid = wgs < most ? wgs : most;
  const bool vec = features % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  if (vec)
    hipLaunchKernelGGL((bfht_mix_mfma<LB, T, true>), dim3((unsigned)grid), dim3(64 * kMixMfmaWaves), 0, s,
                       static_cast<const T*>(x), static_cast<T*>(out), signs, rows, (int)features);
  else
    hipLaunchKernelGGL((bfht_mix_mfma<LB, T, false>), dim3((unsigned)grid), dim3(64 * kMixMfmaWaves), 0, s,
                       static_cast<const T*>(x), static_cast<T*>(out), signs, rows, (int)features);
  return hipGetLastError();
}

template <class T>
hipError_t launch_mix_mfma_t(int log_size, const void* x, void* out, const float* signs, int64_t rows,
                             int64_t features, hipStream_t s) {
  return log_size == 12 ? launch_mix_mfma_lb<12, T>(x, out, signs, rows, features, s)
                        : launch_mix_mfma_lb<10, T>(x, out, signs, rows, features, s);
}

}  // namespace

bool fht_mix_on_matrix_cores(int dtype, int log_size) {
  return (dtype == kBF16 || dtype == kF16) && (log_size == 10 || log_size == 12);
}

hipError_t launch_fht_mix_mfma(int dtype, const void* x, void* out, const float* signs, int64_t rows,
                               int64_t features, int log_size, hipStream_t s) {
  if (!fht_mix_on_matrix_cores(dtype, log_size)) return hipErrorInvalidValue;
  return dtype == kBF16 ? launch_mix_mfma_t<bf16>(log_size, x, out, signs, rows, features, s)
                        : launch_mix_mfma_t<f16>(log_size, x, out, signs, rows, features, s);
}

}  // namespace lwl
