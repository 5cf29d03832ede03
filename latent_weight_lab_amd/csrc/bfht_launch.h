// Internal interface between the C ABI (bfht_abi.cpp) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace lwl {

enum { kF32 = 0, kF16 = 1, kBF16 = 2 };

// Blocks up to 2^15 are transformed whole by one workgroup; larger ones go
// through the float32 work buffer in tile passes.
constexpr int kWholeBlockMaxLog = 15;

// tile-pass prologues / epilogues
enum { kSrcLatent = 0, kSrcGrad = 1, kSrcWork = 2 };
enum { kDstWork = 0, kDstOut = 1, kDstPartial = 2 };

struct BfhtArgs {
  int dtype;
  const void* src;     // forward: latent; backward: grad_out
  void* dst;           // forward: out slice; backward: grad_latent
  void* work;          // float32 scratch (see workspace sizes in bfht_abi.cpp)
  int64_t n;           // latent size
  int log_block;       // log2(B)
  int64_t first_block; // first block overlapped by [start, stop)
  int64_t nblocks;     // blocks overlapped
  int64_t start, stop;
  uint32_t seed32;
  int layers;
};

hipError_t launch_bfht(const BfhtArgs& a, hipStream_t s, bool forward);

// Matrix-core path for bfloat16 blocks of exactly 2^15 (bfht_mfma.hip).  The
// backward writes one float32 partial row of n values per block into `work`.
bool mfma15_applicable(const BfhtArgs& a);
hipError_t launch_mfma15(const BfhtArgs& a, hipStream_t s, bool forward);
hipError_t launch_sign_words(uint32_t seed32, int64_t block, int layer, int64_t first_word,
                             int64_t nwords, uint32_t* out, hipStream_t s);

struct LinearArgs {
  int dtype;
  const void* x;       // [tokens, in]
  const void* latent;  // [n]
  void* out;           // [tokens, out]
  void* work;          // linear_workspace_bytes(*this) bytes, 256-byte aligned
  int64_t tokens, in_features, out_features, n;
  int log_block;
  int64_t nblocks_w;   // ceil(in*out / B)
  uint32_t seed32;
  int layers;
  float weight_scale;
  int token_splits;
};

// Fused linear limits: the generated block (<= 2^15) and its row layout live
// in LDS; in_features bounds the padded row length.
constexpr int kLinearMaxInFeatures = 32768;
extern const bool kLinearKernelAvailable;
// Shapes the fused kernel (bfht_linear.hip) takes: bf16 blocks of 2^15,
// in_features % 8 == 0 and 528 <= in_features <= 5120 (at most 64 output rows per
// generated block, and their k-major table fits in the LDS).
bool linear_applicable(int dtype, int log_block, int64_t in_features);
int linear_token_splits(const LinearArgs& a);
// Workspace of one call: float32 partial dot products of the rows that
// straddle two blocks, then (for large batches) x re-laid out in MFMA order.
size_t linear_workspace_bytes(const LinearArgs& a);
hipError_t launch_linear(const LinearArgs& a, hipStream_t s);

// Fused latent gradient of BlockFHTLinear (bfht_linear_bwd.hip):
// grad_latent = weight_scale * T^T(grad^T x) with grad^T x formed per block on
// chip.  bf16, B = 2^15, in_features % 16 == 0, at most 4 row tiles per block.
struct LinearBwdArgs {
  const void* grad;    // [tokens, out]
  const void* x;       // [tokens, in]
  void* grad_latent;   // [n], bf16
  void* work;          // linear_bwd_workspace_bytes(*this) bytes, 256-byte aligned
  int64_t tokens, in_features, out_features, n;
  int log_block;
  int64_t nblocks_w;   // ceil(in*out / B)
  uint32_t seed32;
  int layers;
  float weight_scale;
  int token_splits;
};
bool linear_bwd_applicable(int dtype, int log_block, int64_t in_features);
int linear_bwd_token_splits(const LinearBwdArgs& a);
size_t linear_bwd_workspace_bytes(const LinearBwdArgs& a);
hipError_t launch_linear_bwd(const LinearBwdArgs& a, hipStream_t s);

// Fixed-order sum of `rows` float32 partial rows (row r at part + r * stride)
// into dst[0 .. n) of the given dtype (bfht_kernels.hip).
hipError_t launch_block_sum(const float* part, int64_t rows, int64_t stride, int64_t n, void* dst, int dtype,
                            hipStream_t s);

}  // namespace lwl
