// Signed activation FHT: y = (S H S pad(x))[:F] per row, S = diag(signs), H the
// normalized Sylvester Walsh-Hadamard transform of order P = 2^LB >= F.
//
// Reference: FixedFHTMix.forward (examples/nanogpt/model.py:200-218: pad the
// last dimension to P, multiply by the ±1 sign buffer, normalized_fht_last_dim
// (:180-197), multiply by the signs again, keep the first F).  S H S is
// symmetric, so the same kernel computes the backward on the gradient.
//
// P = 4096 (GPT-2's 3072 features padded): bfht_mix_square, one wave per row,
// one LDS exchange (below).  Other sizes: bfht_mix_rows, one row per thread
// group of the whole-block VALU geometry (Geo<LB>), the workgroups looping over
// row groups.  A row stays in the coalesced layout (register r of thread t
// holds position r * TB + t), so it is loaded, signed (a per-thread sign mask
// read once per workgroup) and stored without staging, and the transform starts
// on the register bits and needs one LDS exchange per remaining 5-bit group
// plus one back; where a row fits one wave (P <= 2048) no exchange waits at a
// barrier.  The output may alias the input: bfht_mix_rows writes each position
// from the thread that read it, bfht_mix_square from the row's own wave after
// all of the row's reads.
#include "bfht_block.h"

namespace lwl {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Workgroups of one launch: each loops over row groups, so the sign mask is
// built once per workgroup.
constexpr int64_t kMixMaxGrid = 2048;

template <int LB, class T>
__global__ __launch_bounds__(Geo<LB>::WG) void bfht_mix_rows(const T* x, T* out, const float* __restrict__ signs,
                                                            int64_t rows, int features) {
  using Gm = Geo<LB>;
  __shared__ float smem[Gm::LDS_FLOATS];
  const int gi = threadIdx.x >> Gm::LT;
  const int t = threadIdx.x & (Gm::TB - 1);
  float* lds = smem + (Gm::NG > 1 ? gi * Gm::PADDED : 0);
  // coalesced layout: register r holds position r * TB + t (for TB = 1, the
  // whole row); bit r of the mask = sign of that position
  uint32_t neg = 0;
#pragma unroll
  for (int r = 0; r < Gm::E; ++r) neg |= (uint32_t)(signs[r * Gm::TB + t] < 0.0f) << r;
  auto flip = [&](float v, int r) { return __uint_as_float(__float_as_uint(v) ^ (((neg >> r) & 1u) << 31)); };
  const float scale = inv_sqrt_block<LB>();
  const int64_t groups = (rows + Gm::G - 1) / Gm::G;
  for (int64_t rg = blockIdx.x; rg < groups; rg += gridDim.x) {
    const int64_t row = rg * Gm::G + gi;
    const bool active = row < rows;
    const T* xr = x + (active ? row : 0) * features;
    T* orow = out + row * features;
    float v[Gm::E];
    // loads from a valid index (position 0 of the row stands in for the padding)
    // and a select, so all E loads are in flight at once
#pragma unroll
    for (int r = 0; r < Gm::E; ++r) {
      const int p = r * Gm::TB + t;
      const bool ok = active && p < features;
      const float xv = to_f32(xr[ok ? p : 0]);
      v[r] = flip(ok ? xv : 0.0f, r);
    }
    fht_coalesced<LB, Gm::LE, (Gm::TB <= 64)>(v, lds, t);
    if (active) {
#pragma unroll
      for (int r = 0; r < Gm::E; ++r) {
        const int p = r * Gm::TB + t;
        if (p < features) orow[p] = from_f32<T>(flip(v[r] * scale, r));
      }
    }
  }
}

// Rows of P = 2^LB = E x E with E = 2^(LB/2) lanes of one wave per row (P =
// 1024: two rows per wave; P = 4096: one), E values per lane.  A row starts in
// the coalesced layout (lane t, register r: position r * E + t), is transformed
// over the register bits, crosses LDS once into the run layout (lane t holds
// positions t * E .. t * E + E - 1, LDS slot p + p / E: conflict-free both
// ways), is transformed over the register bits again and is stored from the
// run layout with 16-byte stores.  The row never leaves its wave, so the
// exchange needs no barrier: a wave's LDS accesses are performed in order, and
// the next row's writes come after this row's reads in program order.
template <int LB>
struct MixSquare {
  static constexpr int LE = LB / 2;
  static constexpr int E = 1 << LE;     // values per lane = lanes per row
  static constexpr int B = 1 << LB;
  static constexpr int PADDED = B + E;  // slot of position p: p + p / E
  static constexpr int WG = E == 64 ? 64 : 256;
  static constexpr int G = WG / E;      // rows per workgroup
  static_assert(LB % 2 == 0 && E <= 64, "square rows of one wave at most");
};

// bit r of the result = (signs[pos(r)] < 0), r < E; `sg` spans the P signs
template <int E, class Pos>
__device__ __forceinline__ uint64_t sign_mask(__amdgpu_buffer_rsrc_t sg, Pos pos) {
  uint64_t m = 0;
#pragma unroll
  for (int r = 0; r < E; ++r) m |= (uint64_t)(buf_load<float>(sg, pos(r)) < 0.0f) << r;
  return m;
}

// v[r] negated where bit r of mask is set.  For E = 64 one 64-bit shift gives
// the masks of registers r and r + 32 (the low word's bits shifted into the
// high dword stay below its bit 31).
template <int E>
__device__ __forceinline__ void flip_by_mask(float (&v)[E], uint64_t mask) {
  auto flip = [](float x, uint32_t m) { return __uint_as_float(__float_as_uint(x) ^ (m & 0x80000000u)); };
  if constexpr (E == 64) {
#pragma unroll
    for (int r = 0; r < 32; ++r) {
      uint64_t m;
      asm("v_lshlrev_b64 %0, %1, %2" : "=v"(m) : "v"(31 - r), "v"(mask));
      v[r] = flip(v[r], (uint32_t)m);
      v[r + 32] = flip(v[r + 32], (uint32_t)(m >> 32));
    }
  } else {
#pragma unroll
    for (int r = 0; r < E; ++r) v[r] = flip(v[r], (uint32_t)mask << (31 - r));
  }
}

template <int LB, class T>
__global__ __launch_bounds__(MixSquare<LB>::WG) void bfht_mix_square(const T* x, T* out,
                                                                     const float* __restrict__ signs, int64_t rows,
                                                                     int features, int vec_out) {
  using M = MixSquare<LB>;
  constexpr int E = M::E;
  constexpr int RW = 64 / E;                 // rows per wave
  constexpr int kVec = 16 / (int)sizeof(T);  // values per 16-byte store
  __shared__ float smem[M::G * M::PADDED];
  const int gi = threadIdx.x >> M::LE;
  const int t = threadIdx.x & (E - 1);
  const int hw = (threadIdx.x & 63) >> M::LE;                              // this lane's row within its wave
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave index (uniform)
  float* lds = smem + gi * M::PADDED;
  const auto sg = tile_rsrc(signs, (uint64_t)M::B * 4);
  const uint64_t neg_in = sign_mask<E>(sg, [&](int r) { return r * E + t; });   // coalesced layout
  const uint64_t neg_out = sign_mask<E>(sg, [&](int r) { return t * E + r; });  // run layout
  const float scale = inv_sqrt_block<LB>();
  const int64_t groups = (rows + M::G - 1) / M::G;
  const int rbase = hw * features;  // element offset of this lane's row in the span
  for (int64_t rg = blockIdx.x; rg < groups; rg += gridDim.x) {
    // the wave's rows row0 .. row0 + nr - 1 under one wave-uniform buffer
    // resource each for x and out; rows past the end read 0 / are dropped
    const int64_t row0 = rg * M::G + (int64_t)wv * RW;
    const int64_t left = rows - row0;
    const int nr = left < RW ? (left > 0 ? (int)left : 0) : RW;
    const uint64_t span = (uint64_t)nr * (uint64_t)features * sizeof(T);
    const int64_t first = nr > 0 ? row0 * features : 0;
    const auto xr = tile_rsrc(x + first, span);
    const auto orow = tile_rsrc(out + first, span);
    // lane index opaque per iteration: the addresses derived from it are
    // recomputed (a few adds) instead of held in E registers across the loop
    int tl = t;
    asm volatile("" : "+v"(tl));
    // register r: position r * E + t, element rbase + t + r * E of the span (the
    // register term folds into the loads' offset field)
    const int lb = (rbase + tl) * (int)sizeof(T);
    const int room = features - tl;  // register r holds a row position iff r * E < room
    float v[E];
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const int o = lb + r * E * (int)sizeof(T);
      float xv;
      if constexpr (sizeof(T) == 4)
        xv = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, o, 0, 0));
      else
        xv = to_f32(__builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b16(xr, o, 0, 0)));
      // one row per wave: its buffer ends at the row's end, so the padding reads 0
      v[r] = (RW == 1 || r * E < room) ? xv : 0.0f;
    }
    flip_by_mask<E>(v, neg_in);
    butterflies<E>(v, M::LE);
#pragma unroll
    for (int r = 0; r < E; ++r) lds[r * (E + 1) + tl] = v[r];
    asm volatile("" ::: "memory");  // the reads after the writes (one wave: in order)
#pragma unroll
    for (int r = 0; r < E; ++r) v[r] = lds[tl * (E + 1) + r];
    butterflies<E>(v, M::LE);
#pragma unroll
    for (int r = 0; r < E; ++r) v[r] *= scale;
    flip_by_mask<E>(v, neg_out);
    const int p0 = tl * E;
    if (p0 < features) {  // this lane's run holds positions of the row
      const int ob = (rbase + p0) * (int)sizeof(T);
      if (vec_out && p0 + E <= features) {
#pragma unroll
        for (int c = 0; c < E / kVec; ++c) {
          u32x4 w;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if constexpr (sizeof(T) == 4) {
              w[q] = __float_as_uint(v[c * kVec + q]);
            } else {
              const uint32_t lo = __builtin_bit_cast(uint16_t, from_f32<T>(v[c * kVec + 2 * q]));
              const uint32_t hi = __builtin_bit_cast(uint16_t, from_f32<T>(v[c * kVec + 2 * q + 1]));
              w[q] = lo | (hi << 16);
            }
          }
          __builtin_amdgcn_raw_buffer_store_b128(w, orow, ob + c * 16, 0, 0);
        }
      } else {
#pragma unroll
        for (int r = 0; r < E; ++r) {
          if (p0 + r < features) {
            if constexpr (sizeof(T) == 4) {
              __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[r]), orow, ob + r * 4, 0, 0);
            } else {
              __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f32<T>(v[r])), orow,
                                                    ob + r * 2, 0, 0);
            }
          }
        }
      }
    }
  }
}

template <int LB, class T>
hipError_t launch_mix_square(const void* x, void* out, const float* signs, int64_t rows, int64_t features,
                             hipStream_t s) {
  using M = MixSquare<LB>;
  const int64_t groups = (rows + M::G - 1) / M::G;
  const int64_t grid = groups < kMixMaxGrid ? groups : kMixMaxGrid;
  // 16-byte stores need a 16-byte aligned output and rows of whole 16-byte chunks
  const int vec = ((reinterpret_cast<uintptr_t>(out) & 15) == 0 && (features * (int64_t)sizeof(T)) % 16 == 0) ? 1 : 0;
  hipLaunchKernelGGL((bfht_mix_square<LB, T>), dim3((unsigned)grid), dim3(M::WG), 0, s, static_cast<const T*>(x),
                     static_cast<T*>(out), signs, rows, (int)features, vec);
  return hipGetLastError();
}

template <int LB, class T>
hipError_t launch_mix_lb(const void* x, void* out, const float* signs, int64_t rows, int64_t features,
                         hipStream_t s) {
  using Gm = Geo<LB>;
  const int64_t groups = (rows + Gm::G - 1) / Gm::G;
  const int64_t grid = groups < kMixMaxGrid ? groups : kMixMaxGrid;
  hipLaunchKernelGGL((bfht_mix_rows<LB, T>), dim3((unsigned)grid), dim3(Gm::WG), 0, s, static_cast<const T*>(x),
                     static_cast<T*>(out), signs, rows, (int)features);
  return hipGetLastError();
}

template <class T, int... LBs>
hipError_t dispatch_mix(int LB, const void* x, void* out, const float* signs, int64_t rows, int64_t features,
                        hipStream_t s, std::integer_sequence<int, LBs...>) {
  using Fn = hipError_t (*)(const void*, void*, const float*, int64_t, int64_t, hipStream_t);
  static const Fn table[] = {(LBs == 12 ? &launch_mix_square<12, T> : &launch_mix_lb<LBs, T>)...};
  return table[LB](x, out, signs, rows, features, s);
}

}  // namespace

hipError_t launch_fht_mix(int dtype, const void* x, void* out, const float* signs, int64_t rows, int64_t features,
                          int log_size, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  if (log_size < 0 || log_size > kTileLog) return hipErrorInvalidValue;
  if (fht_mix_on_matrix_cores(dtype, log_size))
    return launch_fht_mix_mfma(dtype, x, out, signs, rows, features, log_size, s);
  const auto seq = std::make_integer_sequence<int, kTileLog + 1>{};
  switch (dtype) {
    case kF32: return dispatch_mix<float>(log_size, x, out, signs, rows, features, s, seq);
    case kF16: return dispatch_mix<f16>(log_size, x, out, signs, rows, features, s, seq);
    case kBF16: return dispatch_mix<bf16>(log_size, x, out, signs, rows, features, s, seq);
  }
  return hipErrorInvalidValue;
}

}  // namespace lwl
