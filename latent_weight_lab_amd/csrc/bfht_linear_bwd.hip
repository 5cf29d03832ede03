// Fused latent gradient of BlockFHTLinear (bf16, block 2^15):
//
//   grad_latent = weight_scale * sum_b T_b^T (grad_weight[b*B : (b+1)*B]),
//   grad_weight = grad^T @ x   ([out, in], flattened row-major = block positions)
//
// (reference latent_weight_lab/block_fht.py:339-352: grad_weight = g^T x in
// HBM as bf16, then block_fht_grad_latent).  Three steps:
//
// 1. bfht_wgrad_gemm: grad_weight in float32 as S token-split partial sums,
//    P_s = g[T_s]^T x[T_s], on v_mfma_f32_32x32x16_bf16.  Both operands are
//    stored token-major (g [tokens, out], x [tokens, in]) while the MFMA wants
//    8 consecutive tokens per lane, so tiles go to LDS as they are (16-byte
//    global loads along the feature dimension, rows of 64 tokens) and come out
//    through ds_read_b64_tr_b16, which transposes 16-bit elements across the
//    16 lanes of a group: lane j of a group receives element (j & 3) of the
//    8-byte reads of lanes 4e + (j >> 2), e = 0..3.  A lane group reading rows
//    k0 .. k0 + 3 at features f0 + 4 (lane & 3) therefore leaves lane j with
//    feature f0 + j at tokens k0 .. k0 + 3: half of an MFMA operand.
//    Workgroup tile 256 (out) x 128 (in), 8 waves of 64 x 64, token steps of
//    64 double-buffered in LDS with one barrier per step, the operands of the
//    next k step read while the current one multiplies; workgroups are
//    numbered so that consecutive tiles run on the same XCD (shared L2), tile
//    order minor in the dimension with fewer tiles.  The split count fills the
//    chip (tiles x splits ~ 256 workgroups).
// 2. bfht_wgrad_sum: gw = bf16(weight_scale * sum_s P_s), the partials summed
//    in a fixed order and rounded once (the reference's grad_weight is bf16;
//    the scale, which it applies to the latent gradient, commutes with the
//    linear transform), zero-padded to whole blocks.
// 3. The generator's own backward on gw (launch_bfht: the matrix-core adjoint
//    chain per block, then the fixed-order block sum), so the result does not
//    depend on timing.
#include <algorithm>

#include "bfht_mfma_chain.h"

namespace lwl {
namespace {

using namespace mfma15;

typedef __bf16 bf16x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

constexpr int kBM = 256;               // grad_weight rows (out features) per tile
constexpr int kBN = 128;               // grad_weight columns (in features) per tile
constexpr int kBK = 64;                // tokens per step
constexpr int kGemmThreads = 512;      // 8 waves: 4 (rows) x 2 (columns) of 64 x 64
constexpr int kGPitch = kBM + 32;      // bf16 per LDS row of the g tile (576 bytes)
constexpr int kXPitch = kBN + 32;      // bf16 per LDS row of the x tile (320 bytes)
constexpr int kGStage = kBK * kGPitch * 2;
constexpr int kXStage = kBK * kXPitch * 2;
constexpr int kStage = kGStage + kXStage;
constexpr int kGemmLds = 2 * kStage;   // 112 KiB
constexpr int kGChunks = kBK * kBM / 8 / kGemmThreads;  // 16-byte chunks per thread per step: 4
constexpr int kXChunks = kBK * kBN / 8 / kGemmThreads;  // 2
constexpr uint32_t kOff = 0x80000000u;  // buffer offset that reads 0 and drops stores
// Row pitches of 144 / 80 dwords: the four rows k0 .. k0 + 3 of a transposed
// read start 16 banks apart, so 32 lanes (two groups, 64 bytes per row) cover
// all 64 banks once.
static_assert((kGPitch / 2) % 64 == 16 && (kXPitch / 2) % 64 == 16, "transposed reads must not conflict");

__device__ __forceinline__ u32x2v read_tr(const unsigned char* lds, int byte_off) {
  typedef __attribute__((address_space(3))) bf16x4v lds_v;
  lds_v* p = (lds_v*)((__attribute__((address_space(3))) unsigned char*)lds + byte_off);
  return __builtin_bit_cast(u32x2v, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(p));
}

// 8 features f .. f + 7 of token row t of a [tokens, ld] bf16 matrix (zero
// past `rows` or `cols`): one 16-byte load (kVec: ld % 8 == 0, base 16-byte
// aligned), else 8 element loads.
template <bool kVec>
__device__ __forceinline__ u32x4 load_chunk(const __amdgpu_buffer_rsrc_t r, int t, int f, int rows, int cols,
                                            int ld) {
  if constexpr (kVec) {
    const bool ok = t < rows && f < cols;  // cols % 8 == 0: a chunk is all in or all out
    return __builtin_amdgcn_raw_buffer_load_b128(r, ok ? (t * ld + f) * 2 : (int)kOff, 0, 0);
  } else {
    u32x4 v;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const bool ok0 = t < rows && f + e < cols, ok1 = t < rows && f + e + 1 < cols;
      const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(r, ok0 ? (t * ld + f + e) * 2 : (int)kOff, 0, 0);
      const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(r, ok1 ? (t * ld + f + e + 1) * 2 : (int)kOff, 0, 0);
      v[e >> 1] = (lo & 0xffffu) | (hi << 16);
    }
    return v;
  }
}

// Partial sums P_s[o][i] = sum over the split's tokens of g[t][o] x[t][i],
// float32, row-major with row length in_f, split s at part + s * pstride.
template <bool kVecG, bool kVecX>
__global__ __launch_bounds__(kGemmThreads) void bfht_wgrad_gemm(const __bf16* __restrict__ g,
                                                                const __bf16* __restrict__ x,
                                                                float* __restrict__ part, int tokens, int out_f,
                                                                int in_f, int tiles_o, int tiles_i, int splits,
                                                                int steps_per_split, int64_t pstride) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kGemmLds];
  // XCD-aware numbering: the hardware deals workgroups to the 8 XCDs in turn
  // (bid % 8); logical ids run consecutively within an XCD
  const int nwg = tiles_o * tiles_i * splits;
  const int bid = blockIdx.x, xcd = bid & 7, q = nwg >> 3, rem = nwg & 7;
  const int logical = (xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q) + (bid >> 3);
  const int ntiles = tiles_o * tiles_i;
  const int split = logical / ntiles, tile = logical % ntiles;
  int to, ti;
  if (tiles_i >= tiles_o) {
    ti = tile / tiles_o;
    to = tile % tiles_o;
  } else {
    to = tile / tiles_i;
    ti = tile % tiles_i;
  }
  const int o0 = to * kBM, i0 = ti * kBN;
  const int steps = (tokens + kBK - 1) / kBK;
  const int s_first = split * steps_per_split;
  const int s_last = (s_first + steps_per_split < steps) ? s_first + steps_per_split : steps;
  const int t_end = (s_last * kBK < tokens) ? s_last * kBK : tokens;  // tokens of this split end here

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const auto g_r = rsrc(g, (uint32_t)((int64_t)tokens * out_f * 2));
  const auto x_r = rsrc(x, (uint32_t)((int64_t)tokens * in_f * 2));

  // global -> register -> LDS: g chunk c = tid + 512 h (row c / 32, features 8 (c % 32)),
  // x chunk c = tid + 512 h (row c / 16, features 8 (c % 16))
  u32x4 gr[kGChunks], xr[kXChunks];
  auto load_step = [&](int s) {
    const int t0 = s * kBK;
#pragma unroll
    for (int h = 0; h < kGChunks; ++h) {
      const int c = tid + kGemmThreads * h;
      gr[h] = load_chunk<kVecG>(g_r, t0 + (c >> 5), o0 + 8 * (c & 31), t_end, out_f, out_f);
    }
#pragma unroll
    for (int h = 0; h < kXChunks; ++h) {
      const int c = tid + kGemmThreads * h;
      xr[h] = load_chunk<kVecX>(x_r, t0 + (c >> 4), i0 + 8 * (c & 15), t_end, in_f, in_f);
    }
  };
  auto store_step = [&](int stage) {
    unsigned char* sg = lds + stage * kStage;
    unsigned char* sx = sg + kGStage;
#pragma unroll
    for (int h = 0; h < kGChunks; ++h) {
      const int c = tid + kGemmThreads * h;
      *reinterpret_cast<u32x4*>(sg + ((c >> 5) * kGPitch + 8 * (c & 31)) * 2) = gr[h];
    }
#pragma unroll
    for (int h = 0; h < kXChunks; ++h) {
      const int c = tid + kGemmThreads * h;
      *reinterpret_cast<u32x4*>(sx + ((c >> 4) * kXPitch + 8 * (c & 15)) * 2) = xr[h];
    }
  };

  // transposed-read addresses within a stage (bytes): lane group G = lane / 16
  // supplies MFMA lanes 16 G .. 16 G + 15 (row / column 16 (G & 1) + j of a
  // 32-wide operand, tokens 8 (G >> 1) + 0..7 of a 16-token k step)
  const int j = lane & 15, G = lane >> 4;
  const int krow = 8 * (G >> 1) + (j >> 2);     // + 16 kk + 4 r
  const int fcol = 16 * (G & 1) + 4 * (j & 3);  // + 32 (tile within the wave)
  const int wo = wave >> 1, wi = wave & 1;
  const int a_off = (krow * kGPitch + wo * 64 + fcol) * 2;
  const int b_off = kGStage + (krow * kXPitch + wi * 64 + fcol) * 2;

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  // A operand (g rows) and B operand (x columns) of k step kk: two transposed
  // reads each, tokens 0-3 and 4-7 of the lane's eight
  auto read_ops = [&](const unsigned char* st, int kk, u32x4 (&a)[2], u32x4 (&b)[2]) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const u32x2v lo = read_tr(st, a_off + ((16 * kk) * kGPitch + 32 * m) * 2);
      const u32x2v hi = read_tr(st, a_off + ((16 * kk + 4) * kGPitch + 32 * m) * 2);
      a[m] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
#pragma unroll
    for (int nn = 0; nn < 2; ++nn) {
      const u32x2v lo = read_tr(st, b_off + ((16 * kk) * kXPitch + 32 * nn) * 2);
      const u32x2v hi = read_tr(st, b_off + ((16 * kk + 4) * kXPitch + 32 * nn) * 2);
      b[nn] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  };
  auto mfmas = [&](const u32x4 (&a)[2], const u32x4 (&b)[2]) {
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) acc[m][nn] = mfma(a[m], b[nn], acc[m][nn]);
  };

  if (s_first < s_last) {
    load_step(s_first);
    store_step(0);
  }
  __syncthreads();
  for (int s = s_first; s < s_last; ++s) {
    const int cur = (s - s_first) & 1;
    const bool more = s + 1 < s_last;
    if (more) load_step(s + 1);  // in flight while this step multiplies
    const unsigned char* st = lds + cur * kStage;
    // operands of k step kk + 1 are read while the MFMAs of kk run (two register
    // sets; the scheduling barriers keep the compiler from folding them into one)
    u32x4 a0[2], b0[2], a1[2], b1[2];
    read_ops(st, 0, a0, b0);
    read_ops(st, 1, a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    read_ops(st, 2, a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    read_ops(st, 3, a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(a1, b1);
    if (more) store_step(cur ^ 1);  // that stage was last read before the previous barrier
    __syncthreads();
  }

  // D[row m][col n] of a 32 x 32 tile: lane holds n = lane % 32, registers
  // e = 0..15 at m = 8 (e / 4) + 4 (lane / 32) + e % 4
  float* ps = part + (int64_t)split * pstride;
  const int n_l = lane & 31, r_l = 4 * (lane >> 5);
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int nn = 0; nn < 2; ++nn) {
      const int col = i0 + wi * 64 + 32 * nn + n_l;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = o0 + wo * 64 + 32 * m + 8 * (e >> 2) + r_l + (e & 3);
        if (row < out_f && col < in_f) ps[(int64_t)row * in_f + col] = acc[m][nn][e];
      }
    }
}

// grad_weight for the adjoint: gw[q] = bf16(scale * sum_s P_s[q]) in a fixed
// order of s, zero for size <= q < total (whole blocks); 8 positions per thread.
__global__ __launch_bounds__(256) void bfht_wgrad_sum(const float* __restrict__ part, int splits, int64_t pstride,
                                                      int64_t size, int64_t total, float scale,
                                                      __bf16* __restrict__ gw) {
  const int64_t q = 8 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
  if (q >= total) return;
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
  if (q < size) {
    const int off = (int)(q * 4);  // pstride * 4 < 2^31 (host check)
    for (int sb = 0; sb < splits; sb += 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {  // partials past the last read 0 (empty buffer range)
        const auto p_r = rsrc(part + (int64_t)(sb + u) * pstride, sb + u < splits ? (uint32_t)(pstride * 4) : 0u);
        s0 += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(p_r, off, 0, 0));
        s1 += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(p_r, off + 16, 0, 0));
      }
    }
    if (q + 8 > size) {  // straddles the end of grad_weight (the partials' padding is not written)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (q + e >= size) s0[e] = 0.f;
        if (q + 4 + e >= size) s1[e] = 0.f;
      }
    }
  }
  *reinterpret_cast<u32x4*>(gw + q) = u32x4{pk(scale * s0[0], scale * s0[1]), pk(scale * s0[2], scale * s0[3]),
                                            pk(scale * s1[0], scale * s1[1]), pk(scale * s1[2], scale * s1[3])};
}

struct BwdPlan {
  int tiles_o, tiles_i, splits, steps_per_split;
  int64_t pstride;  // floats between partials (in * out rounded up to 64)
  int64_t total;    // whole blocks of grad_weight: nblocks * B
  size_t part_bytes, gw_bytes, rows_bytes;
};

BwdPlan bwd_plan(const LinearBwdArgs& a) {
  BwdPlan p;
  p.tiles_o = (int)((a.out_features + kBM - 1) / kBM);
  p.tiles_i = (int)((a.in_features + kBN - 1) / kBN);
  const int64_t tiles = (int64_t)p.tiles_o * p.tiles_i;
  const int64_t steps = (a.tokens + kBK - 1) / kBK;
  int64_t want = tiles >= 256 ? 1 : 256 / tiles;  // fill the 256 CUs
  if (want > steps) want = steps;
  if (want < 1) want = 1;
  p.steps_per_split = (int)((steps + want - 1) / want);
  p.splits = p.steps_per_split > 0 ? (int)((steps + p.steps_per_split - 1) / p.steps_per_split) : 1;
  if (p.splits < 1) p.splits = 1;
  const int64_t size = a.in_features * a.out_features;
  p.pstride = (size + 63) / 64 * 64;
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  p.total = a.nblocks_w * kB;
  p.part_bytes = al((size_t)p.splits * (size_t)p.pstride * 4);
  p.gw_bytes = al((size_t)p.total * 2);
  // the backward's per-block partial rows (bf16 rows padded to 8 values on the
  // matrix cores; float32 rows of n on the other whole-block kernels)
  const size_t row = std::max((size_t)a.n * 4, (size_t)mfma15_part_stride(a.n) * 2);
  p.rows_bytes = al((size_t)a.nblocks_w * row);
  return p;
}

}  // namespace

bool linear_bwd_applicable(int dtype, int log_block, int64_t in_features) {
  return dtype == kBF16 && log_block == mfma15::kLog && in_features > 0;
}

int linear_bwd_token_splits(const LinearBwdArgs& a) { return bwd_plan(a).splits; }

size_t linear_bwd_workspace_bytes(const LinearBwdArgs& a) {
  const BwdPlan p = bwd_plan(a);
  return p.part_bytes + p.gw_bytes + p.rows_bytes;
}

hipError_t launch_linear_bwd(const LinearBwdArgs& a, hipStream_t s) {
  const BwdPlan p = bwd_plan(a);
  auto* base = (unsigned char*)a.work;
  float* part = (float*)base;
  auto* gw = (__bf16*)(base + p.part_bytes);
  void* rows = base + p.part_bytes + p.gw_bytes;
  const bool vec_g = a.out_features % 8 == 0 && (uintptr_t)a.grad % 16 == 0;
  const bool vec_x = a.in_features % 8 == 0 && (uintptr_t)a.x % 16 == 0;
  const dim3 grid((unsigned)((int64_t)p.tiles_o * p.tiles_i * p.splits)), block(kGemmThreads);
#define LWL_WGRAD(VG, VX)                                                                                        \
  hipLaunchKernelGGL((bfht_wgrad_gemm<VG, VX>), grid, block, 0, s, (const __bf16*)a.grad, (const __bf16*)a.x,   \
                     part, (int)a.tokens, (int)a.out_features, (int)a.in_features, p.tiles_o, p.tiles_i,         \
                     p.splits, p.steps_per_split, p.pstride)
  if (vec_g && vec_x) LWL_WGRAD(true, true);
  else if (vec_g) LWL_WGRAD(true, false);
  else if (vec_x) LWL_WGRAD(false, true);
  else LWL_WGRAD(false, false);
#undef LWL_WGRAD
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(bfht_wgrad_sum, dim3((unsigned)((p.total / 8 + 255) / 256)), dim3(256), 0, s, part, p.splits,
                     p.pstride, a.in_features * a.out_features, p.total, a.weight_scale, gw);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // the generator's backward over whole blocks: adjoint chains, then the fixed-order block sum
  BfhtArgs b{};
  b.dtype = kBF16;
  b.src = gw;
  b.dst = a.grad_latent;
  b.work = rows;
  b.n = a.n;
  b.log_block = mfma15::kLog;
  b.first_block = 0;
  b.nblocks = a.nblocks_w;
  b.start = 0;
  b.stop = p.total;
  b.seed32 = a.seed32;
  b.layers = a.layers;
  return launch_bfht(b, s, false);
}

}  // namespace lwl
