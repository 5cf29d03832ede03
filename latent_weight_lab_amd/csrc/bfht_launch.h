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

// The tile-pass forward runs its passes over groups of blocks whose work
// buffer is at most 128 MiB (at least one block): a group's passes then find
// more of the buffer in the 256 MB last-level cache (config 3, 2^26
// coordinates in two groups, same box: 0.421 -> 0.397-0.403 ms at 2^23
// blocks, 2^20 unchanged within the spread), the workspace halves, and
// quarter-size groups leave too few tiles per CU (0.42 / 0.44 ms).  The
// backward, whose last pass sums across blocks, does not gain and is not split.
constexpr int64_t kTileGroupBytes = (int64_t)128 << 20;
inline int64_t tile_group_blocks(int log_block) {
  const int64_t b = kTileGroupBytes >> (log_block + 2);
  return b > 0 ? b : 1;
}

// tile-pass prologues / epilogues
enum { kSrcLatent = 0, kSrcGrad = 1, kSrcWork = 2 };
enum { kDstWork = 0, kDstOut = 1, kDstSum = 2 };

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

// Device address of the no-allocation entry's scratch array on the device of
// stream s (bfht_noalloc.hip), or nullptr with the HIP error in *err.
void* noalloc_scratch(hipStream_t s, hipError_t* err);

// Matrix-core path for bfloat16 blocks of exactly 2^15 (bfht_mfma.hip).  The
// backward writes one float32 partial row of n values per block into `work`.
bool mfma15_applicable(const BfhtArgs& a, bool fwd);
// The matrix-core backward's partial rows: bfloat16, rows of n padded to 8
// elements (16-byte aligned), inside the float32-row workspace.
__host__ __device__ inline int64_t mfma15_part_stride(int64_t n) { return (n + 7) / 8 * 8; }
hipError_t launch_mfma15(const BfhtArgs& a, hipStream_t s, bool forward);
hipError_t launch_sign_words(uint32_t seed32, int64_t block, int layer, int64_t first_word,
                             int64_t nwords, uint32_t* out, hipStream_t s);

// Epilogue of the fused linear (lwl_bfht_linear_forward_ex): the stored value
// is v = scale * acc, then + cscale * (*coef) * xsum[t] (coef set), + base[t, o]
// (base set), + bias[o] (bias set), in float32 in that order.  xsum holds the
// float32 row sums of x (launch_row_sums) when coef is set.
struct LinearEpi {
  const void* bias;   // [out], the I/O dtype
  const void* base;   // [tokens, out], the I/O dtype
  const float* coef;  // one float32 on the device
  const float* xsum;  // [tokens]
  float cscale;
};

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
  int blocks_per_wg;   // generated blocks per workgroup (linear_blocks_per_wg)
  int rows_per_tile;   // > 0: tiles of this many whole rows instead (linear_rows_per_tile)
  int token_splits;
  LinearEpi epi;       // all null: plain out = weight_scale * x @ W^T
};

// Float32 row sums of x [tokens, in] into xsum, one wave per row in a fixed
// order (bfht_linear_small.hip).
hipError_t launch_row_sums(const LinearArgs& a, float* xsum, hipStream_t s);

// Fused linear limits: the generated block (<= 2^15) and its row layout live
// in LDS; in_features bounds the padded row length.
constexpr int kLinearMaxInFeatures = 32768;
extern const bool kLinearKernelAvailable;
// Shapes the fused kernel (bfht_linear.hip) takes: bf16 blocks of 2^15,
// in_features % 8 == 0 and 528 <= in_features <= 5120 (at most 64 output rows per
// generated block, and their k-major table fits in the LDS).
bool linear_applicable(int dtype, int log_block, int64_t in_features);
int linear_blocks_per_wg(const LinearArgs& a);  // needs tokens, in/out features, nblocks_w
int linear_rows_per_tile(const LinearArgs& a);  // needs blocks_per_wg
int linear_token_splits(const LinearArgs& a);     // needs blocks_per_wg, rows_per_tile
// Workspace of one call: float32 partial dot products of the rows that
// straddle two blocks, then (for large batches) x re-laid out in MFMA order.
size_t linear_workspace_bytes(const LinearArgs& a);
hipError_t launch_linear(const LinearArgs& a, hipStream_t s);

// Several fused linears in few launches (bfht_linear.hip): jobs the
// matrix-core kernel takes with one generated block per workgroup (batches
// below its tiled-x size) run in one launch per layer count of up to
// kLinearGroupMax jobs, each job exactly as its single launch computes it
// (same work items, same partial-row sums), with its own `work` (partial rows,
// linear_workspace_bytes, inside one workspace) and at most a bias as epilogue.
constexpr int kLinearGroupMax = 48;  // the table stays below the 4 KiB of kernel arguments
struct LinearGroupJob {
  const __bf16* x;
  const __bf16* latent;
  __bf16* out;
  const __bf16* bias;      // or nullptr
  int32_t tokens, in_f, out_f, n;
  uint32_t seed32;
  float scale;
  int32_t nblocks, pitch, token_split;
  uint32_t partial_off;    // floats from LinearGroupTable::partial
};
struct LinearGroupTable {  // passed by value; prefix counts workgroups, cprefix combine workgroups
  float* partial;          // the lowest of the jobs' `work`
  int32_t count;
  int32_t prefix[kLinearGroupMax + 1];
  int32_t cprefix[kLinearGroupMax + 1];
  LinearGroupJob job[kLinearGroupMax];
};
static_assert(sizeof(LinearGroupTable) <= 4000, "grouped linear table fits the kernel arguments");
bool linear_groupable(const LinearArgs& a);  // shape only; the caller checks the epilogue
// x [tokens, row_bytes] re-laid out in MFMA A-operand order (bfht_linear.hip):
// per 16-token tile and 64-byte step of k, one 1 KiB group of 16-byte chunks,
// chunk (l & 15) + 16 (l >> 4) = bytes 64 s + 16 (l >> 4) .. + 15 of row
// 16 T + (l & 15); rows past tokens and bytes past the row read 0.  row_bytes
// % 16 == 0; the copy takes ceil(tokens / 16) * ceil(row_bytes / 64) KiB.
hipError_t launch_tile_x(const void* x, void* xt, int64_t tokens, int64_t row_bytes, hipStream_t s);
hipError_t launch_linear_grouped(const LinearArgs* jobs, int64_t count, hipStream_t s);

// The reference extension's own fused-linear domain (bfht_linear_small.hip):
// float32 / float16 / bfloat16 latents, B <= 2^14, B % in_features == 0, so no
// row straddles two blocks.  Blocks generated in float32 into LDS and
// contracted there in float32; no workspace.
constexpr int kLinearSmallMaxLog = 14;
bool linear_small_applicable(int dtype, int log_block, int64_t in_features);
int linear_small_token_splits(const LinearArgs& a);  // needs tokens, log_block, nblocks_w
hipError_t launch_linear_small(const LinearArgs& a, hipStream_t s);
// The same domain at batches of kLinearMmMinTokens and more, contracted on the
// matrix cores (bfht_linear_small_mm.hip): blocks of 2^5 .. 2^14, in_features a
// multiple of 32 (16-bit I/O) or 16 (float32) with at least 16 rows per
// 32768-weight (16384 for float32) workgroup tile.  From 16 tokens: the VALU
// kernel's contraction costs ~1.1 us per token (1024 -> 4096, latent 16384:
// 18.4-22.1 us at 8 tokens, 27.2-34.2 at 16), the matrix-core one's call is
// flat (24.7-31.7 us from 8 to 64 tokens).
constexpr int kLinearMmMinLog = 5;
constexpr int64_t kLinearMmMinTokens = 16;
bool linear_small_mm_applicable(const LinearArgs& a);  // needs dtype, log_block, in/out features, tokens
int linear_small_mm_token_splits(const LinearArgs& a);
// From 256 tokens its workspace holds x re-laid out (launch_tile_x); else none.
size_t linear_small_mm_workspace_bytes(const LinearArgs& a);
hipError_t launch_linear_small_mm(const LinearArgs& a, hipStream_t s);

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

// Grouped whole-weight generation and its adjoint: the weight-cache prepare and
// flush of many generators (one per BlockFHTLinear) in a few launches
// (bfht_grouped.cpp plans them).  Each job is one generator over [0, size):
//   forward   dst[i] = W(T(T(gen[i]) * scale))                   (weight dtype W)
//   backward  r = T(T(adjoint(T(src))) * scale); dst = accumulate ? T(dst + r) : r
// with T the latent dtype, i.e. the roundings of the per-generator launch
// followed by torch's `* weight_scale`, `.to(dtype)` and `grad.add_`.
constexpr int kGroupMaxJobs = 32;
struct GroupJob {
  const void* src;   // forward: latent [n]; backward: grad of the weight [size] (weight dtype)
  void* dst;         // forward: weight [size] (weight dtype); backward: grad_latent [n]
  void* part;        // backward: nblocks partial rows of n values, `stride` values apart
  int64_t size;
  int32_t n;
  int32_t stride;    // 128-byte aligned rows: n rounded up to 32 floats or 64 bfloat16
  int32_t part_bf16; // rows are bfloat16 (the matrix-core chain's backward), else float32
  int32_t nblocks;   // ceil(size / B)
  uint32_t seed32;
  int32_t layers;
  int32_t wdtype;    // weight dtype code
  int32_t accumulate;
  float scale;
};
// Passed by value; prefix[j] = first workgroup of job j, prefix[count] = grid.
struct GroupTable {
  int32_t count;
  int32_t prefix[kGroupMaxJobs + 1];
  GroupJob job[kGroupMaxJobs];
};
// Whole-block jobs (B <= 2^15) of one latent dtype, weight dtype and block size
// (bfht_grouped_kernels.hip).
int group_slots_per_wg(int log_block);
hipError_t launch_block_grouped(const GroupTable& g, int dtype, int wdtype, int log_block, hipStream_t s,
                                bool fwd);
// bfloat16 jobs of block 2^15 and one layer count on the matrix cores.
hipError_t launch_mfma15_grouped(const GroupTable& g, int layers, hipStream_t s, bool fwd);
// Block sums of backward jobs of one latent dtype and one partial-row type
// (prefix in 256-column tiles).
constexpr int kGroupReduceCols = 256;
hipError_t launch_reduce_grouped(const GroupTable& g, int dtype, bool part_bf16, hipStream_t s);

// One generator of a grouped call (validated by the C ABI).
struct WeightJob {
  const void* latent;       // [n], ldtype
  void* weight;             // forward: [size], wdtype
  const void* grad_weight;  // backward: [size], wdtype
  void* grad_latent;        // backward: [n], ldtype
  int64_t n, size;
  int layers;
  uint32_t seed32;
  int ldtype, wdtype;
  float scale;
  int accumulate;
};
constexpr int64_t kGroupMaxGrid = ((int64_t)1 << 31) - 1;  // workgroups of one grouped launch
// Whether the grouped kernels take the job (else *why says what is missing).
bool grouped_job_supported(const WeightJob& j, bool fwd, const char** why);
// Backward workspace: every job's partial rows, each 256-byte aligned.
size_t grouped_workspace_bytes(const WeightJob* jobs, int64_t count);
hipError_t launch_grouped(const WeightJob* jobs, int64_t count, void* work, hipStream_t s, bool fwd);

// Signed activation FHT of `rows` rows of `features` values (bfht_mix.hip):
// out = (S H S pad(x))[:features] per row, H of order 2^log_size, S = diag(signs).
hipError_t launch_fht_mix(int dtype, const void* x, void* out, const float* signs, int64_t rows, int64_t features,
                          int log_size, hipStream_t s);
// float16 / bfloat16 rows of 2^10 or 2^12 run on the matrix cores (bfht_mix_mfma.hip).
bool fht_mix_on_matrix_cores(int dtype, int log_size);
hipError_t launch_fht_mix_mfma(int dtype, const void* x, void* out, const float* signs, int64_t rows,
                               int64_t features, int log_size, hipStream_t s);

}  // namespace lwl
