// Fused latent gradient of BlockFHTLinear (bf16, block 2^15):
//
//   grad_latent = weight_scale * sum_b T_b^T (grad_weight[b*B : (b+1)*B]),
//   grad_weight = grad^T @ x   ([out, in], never written to memory)
//
// (reference latent_weight_lab/block_fht.py:339-352: grad_weight = g^T x in HBM,
// then block_fht_grad_latent).  One workgroup per (generated block b, token
// range): it contracts the block's rows of g^T x over its tokens on
// v_mfma_f32_16x16x32_bf16, rounds the tile to bf16 into LDS in block-position
// order (positions of rows that straddle into a neighbouring block are left to
// that block's workgroup), runs the adjoint chain of bfht_mfma_chain.h on it
// and writes weight_scale times its float32 partial latent row.  The rows of
// all (block, token range) pairs are then summed in a fixed order, so the
// result does not depend on timing.  The transform is linear, so summing the
// per-token-range images after the chain equals transforming their sum.
//
// Both MFMA operands need 8 consecutive tokens per lane, while x and g are
// stored token-major: x is re-laid out once into 16-column x 32-token tiles
// (1 KiB per operand load), g transposed to [out, tokens].
#include "bfht_mfma_chain.h"

namespace lwl {
namespace {

using namespace mfma15;

typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kTokStep = 32;  // tokens per MFMA k step

__device__ __forceinline__ f32x4v mfma16(u32x4 a, u32x4 b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

struct BwdPlan {
  int64_t steps;   // token steps of 32 (tokens zero-padded)
  int64_t itiles;  // in_features / 16
  size_t partial_bytes, xt_bytes, gt_bytes;
};

BwdPlan bwd_plan(const LinearBwdArgs& a) {
  BwdPlan p;
  p.steps = (a.tokens + kTokStep - 1) / kTokStep;
  p.itiles = a.in_features / 16;
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  p.partial_bytes = al((size_t)a.nblocks_w * (size_t)a.token_splits * (size_t)a.n * 4);
  p.xt_bytes = al((size_t)p.itiles * (size_t)p.steps * 1024);
  p.gt_bytes = al((size_t)a.out_features * (size_t)p.steps * kTokStep * 2);
  return p;
}

// x [tokens, in] -> xt: for column tile I and token step s, 64 16-byte chunks,
// chunk (l16 + 16*kq) = x[32 s + 8 kq .. +7][16 I + l16] (zero past the end).
// Grid (steps, ceil(in / 128)); each workgroup moves a 32-token x 128-column
// tile through LDS: row-contiguous loads, chunk-contiguous stores.
__global__ __launch_bounds__(256) void bwd_tile_x(const __bf16* __restrict__ x, u32x4* __restrict__ xt,
                                                  int tokens, int in_f, int steps, int itiles) {
  constexpr int kPitch = 136;  // bf16 per LDS row (128 + 8: rows start on different banks)
  __shared__ __attribute__((aligned(16))) uint16_t tile[kTokStep * kPitch];
  const int s = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
  const auto x_r = rsrc(x, (uint32_t)((int64_t)tokens * in_f * 2));
  {
    const int r = t >> 3, cg = t & 7;  // token row, 16-column group
    const int tok = s * kTokStep + r, col = c * 128 + cg * 16;
    const bool ok = tok < tokens && col < in_f;  // in % 16 == 0: a group is all in or all out
    const int off = ok ? (tok * in_f + col) * 2 : (int)0x80000000;
    const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(x_r, off, 0, 0);
    const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(x_r, ok ? off + 16 : off, 0, 0);
    u32x4* dst = reinterpret_cast<u32x4*>(tile + r * kPitch + cg * 16);
    dst[0] = v0;
    dst[1] = v1;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int q = h * 256 + t;                       // chunk of this workgroup's 8 column tiles
    const int il = q >> 6, lane = q & 63;
    const int I = c * 8 + il;
    const int col = il * 16 + (lane & 15), r0 = 8 * (lane >> 4);
    u32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[e] = (uint32_t)tile[(r0 + 2 * e) * kPitch + col] | ((uint32_t)tile[(r0 + 2 * e + 1) * kPitch + col] << 16);
    if (I < itiles) xt[((int64_t)I * steps + s) * 64 + lane] = v;
  }
}

// g [tokens, out] -> gt [out, steps * 32] (token-contiguous rows, zero-padded).
// Grid (steps, ceil(out / 128)); a 32-token x 128-row tile through LDS.
__global__ __launch_bounds__(256) void bwd_transpose_g(const __bf16* __restrict__ g, __bf16* __restrict__ gt,
                                                       int tokens, int out_f, int steps) {
  constexpr int kPitch = 130;  // bf16 per LDS row (odd word pitch)
  __shared__ uint16_t tile[kTokStep * kPitch];
  const int s = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
  const auto g_r = rsrc(g, (uint32_t)((int64_t)tokens * out_f * 2));
#pragma unroll
  for (int h = 0; h < 16; ++h) {  // element (row r, column o): consecutive threads, consecutive o
    const int idx = h * 256 + t;
    const int r = idx >> 7, ol = idx & 127;
    const int tok = s * kTokStep + r, o = c * 128 + ol;
    const bool ok = tok < tokens && o < out_f;
    tile[r * kPitch + ol] = __builtin_amdgcn_raw_buffer_load_b16(g_r, ok ? (tok * out_f + o) * 2 : (int)0x80000000,
                                                                 0, 0);
  }
  __syncthreads();
  const int64_t pitch = (int64_t)steps * kTokStep;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int q = h * 256 + t;
    const int ol = q >> 2, kq = q & 3;  // row o, token group of 8
    const int o = c * 128 + ol;
    u32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[e] = (uint32_t)tile[(8 * kq + 2 * e) * kPitch + ol] | ((uint32_t)tile[(8 * kq + 2 * e + 1) * kPitch + ol] << 16);
    if (o < out_f) *reinterpret_cast<u32x4*>(gt + o * pitch + s * kTokStep + 8 * kq) = v;
  }
}

// Main kernel.  NT row tiles of 16 per block (rows o_first .. o_last), IC
// column tiles per wave per pass (NT * IC <= 9 keeps accumulators and two
// steps of operands in registers): wave w owns column tiles w, w + 8, w + 16,
// ... and takes them IC at a time; each pass streams the workgroup's token
// steps once (x tiles are read once per workgroup in total).
template <int L, int NT, int IC>
__global__ __launch_bounds__(kThreads) void bfht_linear_bwd_mfma15(const u32x4* __restrict__ xt,
                                                                   const __bf16* __restrict__ gt,
                                                                   float* __restrict__ partial, int tokens,
                                                                   int in_f, int out_f, int n, int steps,
                                                                   int itiles, uint32_t seed32, float scale,
                                                                   int token_split) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kChainLdsBytes];
  const int64_t block = blockIdx.x / token_split;
  const int split = blockIdx.x % token_split;
  const int64_t size = (int64_t)in_f * out_f;
  const int64_t g0 = block * kB;
  const int64_t g1 = (g0 + kB < size) ? g0 + kB : size;
  const int o_first = (int)(g0 / in_f);
  const int o_last = (int)((g1 - 1) / in_f);
  const int first_off = (int)((int64_t)o_first * in_f - g0);  // in (-in, 0]
  const int per_split = (steps + token_split - 1) / token_split;
  const int s0 = split * per_split;
  const int s1 = (s0 + per_split < steps) ? s0 + per_split : steps;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, kq = lane >> 4;
  const int64_t pitch = (int64_t)steps * kTokStep;
  const auto x_r = rsrc(xt, (uint32_t)((int64_t)itiles * steps * 1024));
  const auto g_r = rsrc(gt, (uint32_t)((int64_t)out_f * pitch * 2));
  constexpr uint32_t kOff = 0x80000000u;  // voffset that reads 0

  // bf16 image of this block's slice of grad_weight (positions 0 .. B-1), in
  // exchange buffer 0; positions no row of this workgroup covers stay 0
  uint16_t* img = reinterpret_cast<uint16_t*>(lds);
  for (int i = threadIdx.x; i < kB / 8; i += kThreads) reinterpret_cast<u32x4*>(img)[i] = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();

  // A operand rows (one per row tile): gt row o_first + 16 nt + l16, 8 tokens at 8 kq
  uint32_t ga[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int o = o_first + 16 * nt + l16;
    ga[nt] = o < out_f ? (uint32_t)((o * pitch + 8 * kq) * 2) : kOff;
  }
  const int ipw = (itiles - wave + kWaves - 1) / kWaves;  // this wave's column tiles
  for (int j0 = 0; j0 < ipw; j0 += IC) {
    uint32_t xb[IC];
#pragma unroll
    for (int j = 0; j < IC; ++j) {
      const int I = wave + kWaves * (j0 + j);
      xb[j] = (j0 + j < ipw) ? (uint32_t)(((int64_t)I * steps * 64 + lane) * 16) : kOff;
    }
    f32x4v acc[NT][IC];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int j = 0; j < IC; ++j) acc[nt][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
    // one step of prefetch: operands of step s + 1 load while step s multiplies
    auto load = [&](int s, u32x4 (&a)[NT], u32x4 (&b)[IC]) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        a[nt] = __builtin_amdgcn_raw_buffer_load_b128(g_r, (int)ga[nt], s * kTokStep * 2, 0);
#pragma unroll
      for (int j = 0; j < IC; ++j) b[j] = __builtin_amdgcn_raw_buffer_load_b128(x_r, (int)xb[j], s * 1024, 0);
    };
    u32x4 a0[NT], b0[IC], a1[NT], b1[IC];
    if (s0 < s1) load(s0, a0, b0);
    for (int s = s0; s < s1; s += 2) {
      if (s + 1 < s1) load(s + 1, a1, b1);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int j = 0; j < IC; ++j) acc[nt][j] = mfma16(a0[nt], b0[j], acc[nt][j]);
      if (s + 1 >= s1) break;
      if (s + 2 < s1) load(s + 2, a0, b0);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int j = 0; j < IC; ++j) acc[nt][j] = mfma16(a1[nt], b1[j], acc[nt][j]);
    }
    // D[m = 4 kq + r][n = l16] = grad_weight[o_first + 16 nt + m][16 I + n] over this token range;
    // block position of (row o_first + ol, column i) = ol * in + i + first_off
#pragma unroll
    for (int j = 0; j < IC; ++j) {
      if (j0 + j >= ipw) continue;
      const int i = 16 * (wave + kWaves * (j0 + j)) + l16;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ol = 16 * nt + 4 * kq + r;
          const int p = ol * in_f + i + first_off;
          if (ol <= o_last - o_first && p >= 0 && p < kB)
            img[p] = __builtin_bit_cast(uint16_t, (__bf16)acc[nt][j][r]);
        }
    }
  }
  __syncthreads();

  // adjoint chain on the image: D_0 H D_1 ... H D_L, then scale * D_0 row of n
  const Ctx c = make_ctx(seed32, block);
  u32x4 src[kTiles][2];
  load_source(c, [&](int p) -> u32x4 { return *reinterpret_cast<const u32x4*>(img + p); }, src);
  __syncthreads();  // the image is exchange buffer 0, rewritten by the first layer
  f32x16 acc[kTiles];
  uint32_t nw[4];
  run_chain<L>(acc, c, lds, src, [](int i) { return L - i; }, nw);
  write_partial_row<L, false>(acc, nw, c, lds, partial + (int64_t)blockIdx.x * n, n, scale);
}

template <int L>
hipError_t launch_bwd_main(const LinearBwdArgs& a, const BwdPlan& p, const u32x4* xt, const __bf16* gt,
                           float* partial, hipStream_t s) {
  const int nt = (int)((kB + a.in_features - 1) / a.in_features + 1 + 15) / 16;
  const dim3 grid((unsigned)(a.nblocks_w * a.token_splits)), block(kThreads);
#define LWL_BWD(NT, IC)                                                                                          \
  hipLaunchKernelGGL((bfht_linear_bwd_mfma15<L, NT, IC>), grid, block, 0, s, xt, gt, partial, (int)a.tokens,    \
                     (int)a.in_features, (int)a.out_features, (int)a.n, (int)p.steps, (int)p.itiles, a.seed32,   \
                     a.weight_scale, a.token_splits)
  switch (nt) {
    case 1: LWL_BWD(1, 8); break;
    case 2: LWL_BWD(2, 4); break;
    case 3: LWL_BWD(3, 3); break;
    case 4: LWL_BWD(4, 2); break;
    default: return hipErrorInvalidValue;
  }
#undef LWL_BWD
  return hipGetLastError();
}

}  // namespace

bool linear_bwd_applicable(int dtype, int log_block, int64_t in_features) {
  // bf16 chain at B = 2^15; 16-column tiles (in % 16 == 0); at most 4 row tiles of 16 per block
  if (dtype != kBF16 || log_block != mfma15::kLog || in_features % 16 != 0 || in_features > mfma15::kB) return false;
  return ((mfma15::kB + in_features - 1) / in_features + 1 + 15) / 16 <= 4;
}

int linear_bwd_token_splits(const LinearBwdArgs& a) {
  const int64_t steps = (a.tokens + kTokStep - 1) / kTokStep;
  int64_t split = a.nblocks_w >= 256 ? 1 : 256 / a.nblocks_w;
  if (split > steps) split = steps;
  return (int)(split < 1 ? 1 : split);
}

size_t linear_bwd_workspace_bytes(const LinearBwdArgs& a) {
  const BwdPlan p = bwd_plan(a);
  return p.partial_bytes + p.xt_bytes + p.gt_bytes;
}

hipError_t launch_linear_bwd(const LinearBwdArgs& a, hipStream_t s) {
  const BwdPlan p = bwd_plan(a);
  auto* base = (unsigned char*)a.work;
  float* partial = (float*)base;
  auto* xt = (u32x4*)(base + p.partial_bytes);
  auto* gt = (__bf16*)(base + p.partial_bytes + p.xt_bytes);
  hipLaunchKernelGGL(bwd_tile_x, dim3((unsigned)p.steps, (unsigned)((a.in_features + 127) / 128)), dim3(256), 0, s,
                     (const __bf16*)a.x, xt, (int)a.tokens, (int)a.in_features, (int)p.steps, (int)p.itiles);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(bwd_transpose_g, dim3((unsigned)p.steps, (unsigned)((a.out_features + 127) / 128)), dim3(256),
                     0, s, (const __bf16*)a.grad, gt, (int)a.tokens, (int)a.out_features, (int)p.steps);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  switch (a.layers) {
    case 1: e = launch_bwd_main<1>(a, p, xt, gt, partial, s); break;
    case 2: e = launch_bwd_main<2>(a, p, xt, gt, partial, s); break;
    case 3: e = launch_bwd_main<3>(a, p, xt, gt, partial, s); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  return launch_block_sum(partial, a.nblocks_w * a.token_splits, a.n, a.n, a.grad_latent, kBF16, s);
}

}  // namespace lwl
