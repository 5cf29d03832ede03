// Fused BlockFHTLinear forward for the reference extension's own domain:
// float32 / float16 / bfloat16, block B <= 2^14 and B % in_features == 0
// (reference gate latent_weight_lab/block_fht.py:263-273, kernel
// csrc/block_fht_ext_cuda.cu:225-329, launcher :624-681).
//
// out[t, o] = sum_i x[t, i] * (weight_scale * W[o, i]),  W[o, i] = y[o * in + i]
//
// in_features divides B, so every output row lies inside one generated block
// and no row straddles two.  A workgroup owns G consecutive blocks (the slots of
// the whole-block VALU generator: one block of 2^14 per 512-thread workgroup,
// or 256 / (B/32) smaller blocks per 256-thread workgroup) and a range of
// tokens.  It generates its blocks in float32 straight into an LDS weight tile
// (the generator's final stores land in LDS instead of memory, already scaled
// by weight_scale, as the reference scales its shared-memory values), then
// contracts the tile with its tokens: a team of min(in, 64) lanes computes four
// tokens of one output row, lanes striding over k, and sums its lanes with
// butterfly shuffles.  All arithmetic is float32; x and out keep the I/O type.
// The weight never touches memory.
#include "bfht_block.h"

namespace lwl {
namespace {

// LDS window of the generator's stores: global position g of the workgroup's
// tile lands at w[g - base], multiplied by weight_scale.  `range` / call take
// the role of the buffer-resource form of the per-block store (indices outside
// [0, count) are dropped), `at` the element form.
struct LdsRange {
  int first;
  int count;
};
struct LdsWeightStore {
  float* w;
  int64_t base;
  float scale;
  __device__ LdsRange range(int64_t first, int64_t count) const {
    return LdsRange{(int)(first - base), (int)count};
  }
  __device__ void operator()(LdsRange r, int i, float v) const {
    if ((unsigned)i < (unsigned)r.count) w[r.first + i] = v * scale;
  }
  __device__ void whole(LdsRange r, int b, int c, float v) const { w[r.first + b + c] = v * scale; }
  __device__ void at(int64_t i, float v) const { w[i - base] = v * scale; }
};

constexpr int kQuad = 4;  // tokens per team pass
constexpr int kSpan = 8;  // k iterations of a lane whose x loads are in flight together

template <int LB>
struct SmallLinearGeo {
  using Gm = Geo<LB>;
  static constexpr int kTileElems = Gm::G * Gm::B;  // weights generated per workgroup
  static constexpr int kLdsFloats = BlockLds<LB>::FLOATS + kTileElems;
};

template <int LB, class T>
__global__ __launch_bounds__(Geo<LB>::WG) void bfht_linear_small(const T* __restrict__ x,
                                                                 const T* __restrict__ latent, T* __restrict__ out,
                                                                 int tokens, int in_f, int log_in, int out_f, int n,
                                                                 int64_t nblocks, uint32_t seed32, int layers,
                                                                 float scale, int token_split, LinearEpi ep) {
  using Gm = Geo<LB>;
  using SG = SmallLinearGeo<LB>;
  __shared__ float smem[SG::kLdsFloats];
  float* wt = smem + BlockLds<LB>::FLOATS;  // the weight tile, row-major [rows][in]
  const int64_t tile = blockIdx.x;
  const int split = blockIdx.y;
  const int64_t size = (int64_t)in_f * out_f;
  const int64_t base = tile * SG::kTileElems;

  // this split's token quads, and the x of a quad staged in LDS (step 2)
  const int quads = (tokens + kQuad - 1) / kQuad;
  const int per_split = (quads + token_split - 1) / token_split;
  const int q0 = split * per_split;
  const int q1 = q0 + per_split < quads ? q0 + per_split : quads;
  const auto x_r = tile_rsrc(x, (uint64_t)tokens * in_f * sizeof(T));
  const int nstage = kQuad * in_f;
  const bool staged = nstage <= BlockLds<LB>::FLOATS;
  // thread's share i0 + e * WG (e < kSpan) of quad q's staged x (tokens past the batch read 0)
  auto stage_load = [&](int q, int i0, float (&v)[kSpan]) {
#pragma unroll
    for (int e = 0; e < kSpan; ++e) {
      const int i = i0 + e * Gm::WG;
      const int t = q * kQuad + (i >> log_in);
      v[e] = buf_load<T>(x_r, i < nstage && t < tokens ? t * in_f + (i & (in_f - 1)) : -1);
    }
  };
  // When one round of loads stages a quad, the first quad's are issued before
  // the generator runs, which hides their latency.
  const bool prefetch = staged && nstage <= kSpan * Gm::WG && q0 < q1;
  float xpre[kSpan];
  if (prefetch) stage_load(q0, (int)threadIdx.x, xpre);

  // 1. the tile's G blocks (inactive slots past the last block store nothing;
  //    their rows lie past out_features and are never read)
  const int64_t slot = tile * Gm::G + (threadIdx.x >> Gm::LT);
  block_fwd_slot<LB, T>(latent, LdsWeightStore{wt, base, scale}, n, 0, slot, nblocks, 0, size, seed32, layers,
                        smem);
  __syncthreads();

  // 2. rows row0 .. row0 + rows - 1 against this split's token quads
  const int row0 = (int)(base >> log_in);
  const int tile_rows = SG::kTileElems >> log_in;
  const int rows = out_f - row0 < tile_rows ? out_f - row0 : tile_rows;
  if (rows <= 0 || q0 >= q1) return;  // uniform across the workgroup
  const int log_ks = log_in < 6 ? log_in : 6;  // lanes per team: min(in, 64)
  const int ks = 1 << log_ks;
  const int lane = threadIdx.x & 63;
  const int j = lane & (ks - 1);
  const int team = (int)(threadIdx.x >> log_ks);
  const int nteams = Gm::WG >> log_ks;
  const int npairs = (q1 - q0) * rows;
  const auto o_r = tile_rsrc(out, (uint64_t)tokens * out_f * sizeof(T));
  // epilogue terms (uniform); absent inputs get empty resources
  const bool has_xs = ep.xsum != nullptr, has_base = ep.base != nullptr, has_bias = ep.bias != nullptr;
  const float cx = has_xs ? ep.cscale * *ep.coef : 0.f;
  const auto xs_r = tile_rsrc(has_xs ? (const void*)ep.xsum : (const void*)out, has_xs ? (uint64_t)tokens * 4 : 0);
  const auto b_r = tile_rsrc(has_base ? ep.base : (const void*)out, has_base ? (uint64_t)tokens * out_f * sizeof(T) : 0);
  const auto bias_r = tile_rsrc(has_bias ? ep.bias : (const void*)out, has_bias ? (uint64_t)out_f * sizeof(T) : 0);
  // One team pass: rows r, r + rstride, ... (NR of them; those from `rows` on
  // compute on row r and store nothing) against the first NU tokens of quad q
  // (NU = 1 for a quad holding one token, else kQuad).  Lane j adds
  // x[t][k] w[row][k] for k = j, j + ks, ... in that order (x from `xat`),
  // then the team's lanes are summed with butterfly shuffles.  A team's lanes
  // share the pass, so the shuffles only read lanes that run the same
  // iteration.  Every (row, token) sum takes the same additions in the same
  // order whatever NR and NU are.
  auto pass = [&](auto nr_c, auto nu_c, int q, int r, int rstride, auto xat) {
    constexpr int NR = decltype(nr_c)::value, NU = decltype(nu_c)::value;
    const int t0 = q * kQuad;
    const float* wrow[NR];
#pragma unroll
    for (int h = 0; h < NR; ++h) {
      const int rh = r + h * rstride;
      wrow[h] = wt + ((rh < rows ? rh : r) << log_in);
    }
    float acc[NR][NU];
#pragma unroll
    for (int h = 0; h < NR; ++h)
#pragma unroll
      for (int u = 0; u < NU; ++u) acc[h][u] = 0.f;
    // kSpan iterations' loads are issued before their products (the loop's
    // trip count is not known at compile time, so without this each iteration
    // waited out one load's latency); the k order is the same either way
    int k = j;
    for (; k + (kSpan - 1) * ks < in_f; k += kSpan * ks) {
      float xv[kSpan][NU], wv[kSpan][NR];
#pragma unroll
      for (int i = 0; i < kSpan; ++i) {
#pragma unroll
        for (int h = 0; h < NR; ++h) wv[i][h] = wrow[h][k + i * ks];
#pragma unroll
        for (int u = 0; u < NU; ++u) xv[i][u] = xat(t0, u, k + i * ks);
      }
#pragma unroll
      for (int i = 0; i < kSpan; ++i)
#pragma unroll
        for (int h = 0; h < NR; ++h)
#pragma unroll
          for (int u = 0; u < NU; ++u) acc[h][u] += xv[i][u] * wv[i][h];
    }
    for (; k < in_f; k += ks) {
#pragma unroll
      for (int h = 0; h < NR; ++h) {
        const float w = wrow[h][k];
#pragma unroll
        for (int u = 0; u < NU; ++u) acc[h][u] += xat(t0, u, k) * w;
      }
    }
    // the lane sums: each distance's shuffles of every sum in flight together
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
      if (s >= ks) continue;  // uniform
      float sh[NR][NU];
#pragma unroll
      for (int h = 0; h < NR; ++h)
#pragma unroll
        for (int u = 0; u < NU; ++u) sh[h][u] = __shfl_xor(acc[h][u], s, 64);
#pragma unroll
      for (int h = 0; h < NR; ++h)
#pragma unroll
        for (int u = 0; u < NU; ++u) acc[h][u] += sh[h][u];
    }
    if (j == 0) {
      // The epilogue's inputs first, none behind a branch on its term or
      // behind a store that may alias it (either would be waited out on its
      // own): an absent term's buffer is empty and reads 0, and so does index
      // -1 (rows from `rows` on, tokens past the batch), whose store is dropped.
      float xs[NU], bias_o[NR], base_v[NR][NU];
#pragma unroll
      for (int u = 0; u < NU; ++u) xs[u] = cx * buf_load<float>(xs_r, t0 + u < tokens ? t0 + u : -1);
#pragma unroll
      for (int h = 0; h < NR; ++h) {
        const int rh = r + h * rstride, o = row0 + rh;
        bias_o[h] = buf_load<T>(bias_r, rh < rows ? o : -1);
#pragma unroll
        for (int u = 0; u < NU; ++u)
          base_v[h][u] = buf_load<T>(b_r, rh < rows && t0 + u < tokens ? (t0 + u) * out_f + o : -1);
      }
#pragma unroll
      for (int h = 0; h < NR; ++h) {
        const int rh = r + h * rstride;
        if (rh >= rows) continue;  // uniform across the team
        const int o = row0 + rh;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          const int t = t0 + u;
          const int i = t < tokens ? t * out_f + o : -1;  // -1: the store is dropped
          buf_store<T>(linear_epilogue(acc[h][u], has_xs, xs[u], has_base, base_v[h][u], has_bias, bias_o[h]), o_r, i);
        }
      }
    }
  };
  using One = std::integral_constant<int, 1>;
  using Two = std::integral_constant<int, 2>;
  using Quad = std::integral_constant<int, kQuad>;
  if (staged) {
    // Each quad's x rows are staged once in the generator's LDS (its exchange
    // buffers and sign tables, free after the barrier above) and every team
    // reads them there: read from memory, all the workgroup's passes (and all
    // the workgroups of an XCD, at decode batches) ask its L2 for the same
    // few lines.  Tokens past the batch stage as 0.
    float* xs = smem;
    for (int q = q0; q < q1; ++q) {
      if (q > q0) __syncthreads();  // every team has read the previous quad
      for (int i0 = (int)threadIdx.x; i0 < nstage; i0 += kSpan * Gm::WG) {
        float v[kSpan];
        if (prefetch && q == q0) {
#pragma unroll
          for (int e = 0; e < kSpan; ++e) v[e] = xpre[e];
        } else {
          stage_load(q, i0, v);
        }
#pragma unroll
        for (int e = 0; e < kSpan; ++e)
          if (i0 + e * Gm::WG < nstage) xs[i0 + e * Gm::WG] = v[e];
      }
      __syncthreads();
      // two rows per pass (x read once for both); a quad of one token (decode)
      // computes that token alone
      auto xat = [&](int, int u, int kk) { return xs[(u << log_in) + kk]; };
      const bool single = tokens - q * kQuad == 1;
      for (int r = team; r < rows; r += 2 * nteams) {
        if (single)
          pass(Two{}, One{}, q, r, nteams, xat);
        else
          pass(Two{}, Quad{}, q, r, nteams, xat);
      }
    }
  } else {
    for (int pr = team; pr < npairs; pr += nteams) {
      const int q = q0 + pr / rows;
      int xi[kQuad];
#pragma unroll
      for (int u = 0; u < kQuad; ++u) xi[u] = q * kQuad + u < tokens ? (q * kQuad + u) * in_f : -1;  // -1: reads 0
      pass(One{}, Quad{}, q, pr - (pr / rows) * rows, 0,
           [&](int, int u, int kk) { return buf_load<T>(x_r, xi[u] < 0 ? -1 : xi[u] + kk); });
    }
  }
}

// Float32 sums of the rows of x (the fused linear's row-sum term): one wave per
// row, lanes striding over k with eight loads in flight, then a fixed butterfly.
template <class T>
__global__ __launch_bounds__(256) void bfht_row_sums(const T* __restrict__ x, int tokens, int in_f,
                                                     float* __restrict__ xsum) {
  const int t = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // scalar: uniform resource
  if (t >= tokens) return;
  const int lane = threadIdx.x & 63;
  const auto x_r = tile_rsrc(x + (int64_t)t * in_f, (uint64_t)in_f * sizeof(T));  // k >= in_f reads 0
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < in_f; k0 += 8 * 64) {
#pragma unroll
    for (int u = 0; u < 8; ++u) s[u] += buf_load<T>(x_r, k0 + 64 * u + lane);
  }
  float v = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  if (lane == 0) xsum[t] = v;
}

template <int LB, class T>
hipError_t launch_small_lb(const LinearArgs& a, hipStream_t s) {
  using Gm = Geo<LB>;
  const int64_t wtiles = (a.nblocks_w + Gm::G - 1) / Gm::G;
  int log_in = 0;
  while (((int64_t)1 << log_in) < a.in_features) ++log_in;
  hipLaunchKernelGGL((bfht_linear_small<LB, T>), dim3((unsigned)wtiles, (unsigned)a.token_splits), dim3(Gm::WG), 0,
                     s, (const T*)a.x, (const T*)a.latent, (T*)a.out, (int)a.tokens, (int)a.in_features, log_in,
                     (int)a.out_features, (int)a.n, a.nblocks_w, a.seed32, a.layers, a.weight_scale,
                     a.token_splits, a.epi);
  return hipGetLastError();
}

template <class T, int... LBs>
hipError_t dispatch_small(const LinearArgs& a, hipStream_t s, std::integer_sequence<int, LBs...>) {
  using Fn = hipError_t (*)(const LinearArgs&, hipStream_t);
  static const Fn table[] = {&launch_small_lb<LBs, T>...};
  return table[a.log_block](a, s);
}

}  // namespace

bool linear_small_applicable(int dtype, int log_block, int64_t in_features) {
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return false;
  if (log_block < 0 || log_block > kLinearSmallMaxLog || in_features <= 0) return false;
  return (((int64_t)1 << log_block) % in_features) == 0;
}

int linear_small_token_splits(const LinearArgs& a) {
  // Each split regenerates the workgroup's blocks: at least 32 token quads
  // (128 tokens) per split, and no more workgroups than about four per CU.
  const int g = a.log_block >= 5 ? (a.log_block >= 13 ? 1 : 256 >> (a.log_block - 5)) : 256;
  const int64_t wtiles = (a.nblocks_w + g - 1) / g;
  const int64_t quads = (a.tokens + kQuad - 1) / kQuad;
  int64_t split = (quads + 31) / 32;
  const int64_t cap = wtiles >= 1024 ? 1 : (1024 + wtiles - 1) / wtiles;
  if (split > cap) split = cap;
  if (split > 65535) split = 65535;
  return (int)(split < 1 ? 1 : split);
}

hipError_t launch_row_sums(const LinearArgs& a, float* xsum, hipStream_t s) {
  if (a.tokens == 0) return hipSuccess;
  const dim3 grid((unsigned)((a.tokens + 3) / 4)), block(256);
  switch (a.dtype) {
    case kF32: hipLaunchKernelGGL(bfht_row_sums<float>, grid, block, 0, s, (const float*)a.x, (int)a.tokens,
                                  (int)a.in_features, xsum); break;
    case kF16: hipLaunchKernelGGL(bfht_row_sums<f16>, grid, block, 0, s, (const f16*)a.x, (int)a.tokens,
                                  (int)a.in_features, xsum); break;
    case kBF16: hipLaunchKernelGGL(bfht_row_sums<bf16>, grid, block, 0, s, (const bf16*)a.x, (int)a.tokens,
                                   (int)a.in_features, xsum); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_linear_small(const LinearArgs& a, hipStream_t s) {
  using Seq = std::make_integer_sequence<int, kLinearSmallMaxLog + 1>;
  switch (a.dtype) {
    case kF32: return dispatch_small<float>(a, s, Seq{});
    case kF16: return dispatch_small<f16>(a, s, Seq{});
    case kBF16: return dispatch_small<bf16>(a, s, Seq{});
  }
  return hipErrorInvalidValue;
}

}  // namespace lwl
