/*
 * lwl_bfht.h — C ABI of the MI355X (gfx950) BlockFHT library (liblwl_bfht.so).
 *
 * BlockFHT generates a long vector from a short latent: the latent (length n)
 * is zero-padded to B = next_power_of_two(n), and block b of the output is
 *
 *     y_b = D_{b,L} H D_{b,L-1} H ... H D_{b,0} pad(latent)
 *
 * with H the Sylvester-ordered Walsh-Hadamard transform divided by sqrt(B) and
 * D_{b,l} = diag(+-1) taken from one 32-bit hash word per 32 positions:
 * sign(p) = bit (p & 31) of lowbias32(mix(seed, b, l, p >> 5)), set = +1.
 * Output coordinate g lives in block g / B at position g % B.
 *
 * Every entry point is asynchronous on `stream` (a hipStream_t; pass the
 * caller's current stream), never allocates device memory, never synchronizes
 * the host, and is reentrant.  Device buffers are borrowed; scratch memory is
 * passed in as `workspace` (256-byte aligned) of at least the size the
 * matching *_workspace_size() query returns for the same arguments.
 *
 * Return value: LWL_OK (0) or a negative LWL_ERR_* code; lwl_last_error()
 * returns the message of the calling thread's last failure.
 *
 * Element types: the latent, the generated output and their gradients share
 * one dtype (LWL_DTYPE_*).  Arithmetic is float32 (loads and stores in the I/O
 * dtype), with one exception: bfloat16 latents whose block is exactly 2^15 run
 * on the matrix cores, with bfloat16 operands at every radix-32 Walsh stage
 * (three stages per layer, so 9 roundings at 3 layers, ~5e-3 relative L2
 * against a float64 chain) and float32 accumulation.  Each entry point names
 * which of the two it uses.
 */
#ifndef LWL_BFHT_H
#define LWL_BFHT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum lwl_dtype { LWL_DTYPE_F32 = 0, LWL_DTYPE_F16 = 1, LWL_DTYPE_BF16 = 2 };

enum lwl_status {
  LWL_OK = 0,
  LWL_ERR_INVALID = -1,     /* bad argument value (the reference raises ValueError/RuntimeError) */
  LWL_ERR_UNSUPPORTED = -2, /* valid request outside what the kernels implement */
  LWL_ERR_WORKSPACE = -3,   /* workspace missing or smaller than the query returned */
  LWL_ERR_HIP = -4          /* HIP runtime error while launching */
};

/* Largest block size (after padding) the library transforms: 2^23, as the
 * reference's kGlobalMaxBlockSize (csrc/block_fht_ext_cuda.cu:15).  The
 * reference's lower bound 2^5 (.cu:528) is lifted: any n >= 1 works. */
#define LWL_BFHT_MAX_BLOCK_SIZE (1LL << 23)

/* Message of the calling thread's last failure ("" if none). */
const char* lwl_last_error(void);

/* ABI revision of this header; bumped on any signature change. */
int lwl_abi_version(void);

/* ---------------------------------------------------------------- forward
 * Replaces ext.forward (reference csrc/block_fht_ext.cpp:28-38 ->
 * csrc/block_fht_ext_cuda.cu:516-566), called from
 * latent_weight_lab/block_fht.py:170.
 *
 * Writes out[g - start] = y[g] for g in [start, stop), stop - start elements
 * of `dtype`.  Checks (messages follow the reference): 0 <= start <= stop <=
 * output_size ("invalid slice", .cu:524), layers in {1,2,3} (.cu:525),
 * 1 <= latent_size and B <= 2^23 (.cu:528).
 *
 * dtype F32 and F16, and BF16 at blocks other than 2^15: float32 arithmetic,
 * loads/stores in the I/O type.  dtype BF16 at block 2^15 (16385 <= latent_size
 * <= 32768) with a 16-byte aligned latent: matrix cores, bfloat16 operands at
 * each radix-32 stage, float32 accumulation.
 */
size_t lwl_bfht_forward_workspace_size(int64_t latent_size, int64_t output_size, int64_t start,
                                       int64_t stop);
int lwl_bfht_forward(const void* latent, int dtype, int64_t latent_size, int64_t output_size,
                     int64_t layers, int64_t seed, int64_t start, int64_t stop, void* out,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Host-only argument check of lwl_bfht_forward (no GPU needed). */
int lwl_bfht_check_forward(int dtype, int64_t latent_size, int64_t output_size, int64_t layers,
                           int64_t start, int64_t stop);

/* ---------------------------------------------------------------- backward
 * Replaces ext.backward (reference csrc/block_fht_ext.cpp:40-51 ->
 * csrc/block_fht_ext_cuda.cu:568-622), called from block_fht.py:184 and :223.
 *
 * Overwrites grad_latent[0 .. latent_size) with the adjoint of the forward
 * slice applied to grad_out (stop - start elements):
 *     grad_latent[p] = sum_b [D_{b,0} H D_{b,1} ... H D_{b,L} scatter_b(grad_out)][p].
 * The sum over blocks runs in a fixed order (deterministic, unlike the
 * reference's atomicAdd at .cu:221,493).  grad_out and grad_latent have `dtype`.
 * Arithmetic as lwl_bfht_forward (BF16 at block 2^15: matrix cores, bfloat16
 * operands, float32 accumulation, bfloat16 per-block partial rows summed in
 * float32).
 */
size_t lwl_bfht_backward_workspace_size(int64_t latent_size, int64_t output_size, int64_t start,
                                        int64_t stop);
int lwl_bfht_backward(const void* grad_out, int dtype, int64_t latent_size, int64_t output_size,
                      int64_t layers, int64_t seed, int64_t start, int64_t stop, void* grad_latent,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- backward, no allocation
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory or pass a workspace (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): lwl_bfht_backward with the same
 * arguments but no workspace.  Its scratch is a file-scope device array of
 * LWL_BFHT_NOALLOC_SCRATCH_BYTES per GPU (held from first use to process
 * exit); a call whose scratch (lwl_bfht_backward_workspace_size) exceeds it
 * returns LWL_ERR_UNSUPPORTED.  That covers every whole-block backward (B <=
 * 2^15) of up to 256 blocks of 2^15 (config 2 in float32), not the multi-pass
 * blocks' work buffer beyond 32 MiB.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other threads) race.
 * Allocates nothing; results are bit-identical to lwl_bfht_backward.  The
 * first accepted call on each device resolves the array's device address
 * (hipGetSymbolAddress, which may load the library's code object onto the
 * device): make that call outside stream capture (any accepted call does,
 * e.g. one of an empty slice); later calls, captured or not, read the cached
 * address.
 */
#define LWL_BFHT_NOALLOC_SCRATCH_BYTES (32 << 20)
int lwl_bfht_backward_noalloc(const void* grad_out, int dtype, int64_t latent_size, int64_t output_size,
                              int64_t layers, int64_t seed, int64_t start, int64_t stop, void* grad_latent,
                              void* stream);

/* ---------------------------------------------------------------- fused linear
 * Replaces ext.linear_forward (reference csrc/block_fht_ext.cpp:53-67 ->
 * csrc/block_fht_ext_cuda.cu:624-681), called from block_fht.py:274.
 *
 * out[t, o] = weight_scale * sum_i input[t, i] * W[o, i], W[o, i] = y[o * in + i]
 * with y generated from `latent` over size = in_features * out_features.
 * input is row-major [tokens, in_features], out row-major [tokens, out_features],
 * both `dtype`, as the latent.  W is generated on chip, block by block, and
 * contracted there; only the three-block tiles of in_features 3072 from 2048
 * tokens park part of each workgroup's tile in the workspace (the k steps its
 * LDS cannot hold, one staged block).  Unlike the reference (.cu:639-642) any in_features
 * <= B works (rows may straddle blocks; partial rows are summed in a fixed
 * order through the workspace).  B <= 2^15.
 *
 * Two domains:
 *  (a) bfloat16 latents of block 2^15 with in_features % 8 == 0 and
 *      528 <= in_features <= 5120: the generated weight is rounded to bf16 and
 *      the contraction runs on MFMA with float32 accumulation;
 *  (b) the reference extension's own domain (gate block_fht.py:263-273):
 *      float32, float16 or bfloat16, block <= 2^14, block % in_features == 0:
 *      the weight is generated in float32; below 64 tokens it is contracted
 *      in float32 as the reference's kernel does, from 64 tokens on the
 *      matrix cores (float32: exact float32 products; float16 / bfloat16: the
 *      weight rounded to the I/O type, as the reference's fallback rounds it).
 * Other shapes return LWL_ERR_UNSUPPORTED and the caller generates the weight
 * and calls a GEMM, as the reference's fallback does (block_fht.py:263-288).
 * The workspace query has no dtype (as ext.linear_forward has none) and
 * returns the most any dtype needs for the shape: the block-2^15 kernel's
 * partial rows of the rows that straddle its tiles (none where tiles hold whole
 * rows: from 256 tokens, rows of 768 are tiled 64 at a time; from 2048 tokens,
 * rows of 3072 are tiled 32 at a time, three blocks, and each work item keeps
 * the W tiles its LDS cannot hold and one staged block instead, 104 KiB) and,
 * from 256 tokens, a copy of x in MFMA order (in the reference's domain only
 * that copy, float32's being the largest).
 */
size_t lwl_bfht_linear_forward_workspace_size(int64_t tokens, int64_t in_features,
                                              int64_t out_features, int64_t latent_size);
int lwl_bfht_linear_forward(const void* input, const void* latent, int dtype, int64_t tokens,
                            int64_t in_features, int64_t latent_size, int64_t out_features,
                            int64_t layers, int64_t seed, double weight_scale, void* out,
                            void* workspace, size_t workspace_bytes, void* stream);

/* Host-only argument check of lwl_bfht_linear_forward (no GPU needed). */
int lwl_bfht_check_linear_forward(int dtype, int64_t tokens, int64_t in_features,
                                  int64_t latent_size, int64_t out_features, int64_t layers);

/* ---------------------------------------------------------------- fused linear with epilogue
 * Replaces BlockFHTLinear.forward_fused's tail (reference block_fht.py:493-500:
 * the modulation term, the residual base and the bias, each a separate torch op
 * after ext.linear_forward) with the store of the fused kernels:
 *
 *   out[t, o] = ((weight_scale * sum_i input[t, i] * W[o, i]
 *                 + row_sum_scale * (*row_sum_coef) * sum_i input[t, i])
 *                + base[t, o]) + bias[o]
 *
 * summed in float32 in that order (the product, then the row-sum term, then the
 * base, then the bias: the order of the reference's ops, block_fht.py:493-500;
 * no fused multiply-adds) and rounded once to `dtype` (the reference rounds
 * after each op, so results agree to the I/O type's rounding).  Terms
 * whose pointer is NULL are left out; bias [out_features] and base
 * [tokens, out_features] (the residual base's input @ base_weight^T) are in
 * `dtype`; row_sum_coef is one float32 on the device (the module's
 * modulation_alpha * offset, read by the kernel, so the caller never waits on
 * it).  With epilogue NULL this is lwl_bfht_linear_forward, bit for bit.  Same
 * domains and checks; the workspace (query with the same arguments) adds
 * tokens float32 row sums when row_sum_coef is set.
 */
typedef struct lwl_bfht_linear_epilogue {
  const void* bias;          /* [out_features], dtype, or NULL */
  const void* base;          /* [tokens, out_features], dtype, or NULL */
  const float* row_sum_coef; /* one float32 on the device, or NULL */
  double row_sum_scale;      /* host factor of the row-sum term */
} lwl_bfht_linear_epilogue;

size_t lwl_bfht_linear_forward_ex_workspace_size(int dtype, int64_t tokens, int64_t in_features,
                                                 int64_t out_features, int64_t latent_size,
                                                 const lwl_bfht_linear_epilogue* epilogue);
int lwl_bfht_linear_forward_ex(const void* input, const void* latent, int dtype, int64_t tokens,
                               int64_t in_features, int64_t latent_size, int64_t out_features,
                               int64_t layers, int64_t seed, double weight_scale,
                               const lwl_bfht_linear_epilogue* epilogue, void* out, void* workspace,
                               size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- fused linear, grouped
 * Several lwl_bfht_linear_forward calls in few launches (no reference
 * counterpart: the reference calls ext.linear_forward once per matrix,
 * block_fht.py:274, e.g. once per layer of a network in
 * benchmarks/bench_fused_linear_stack.py:31-36).  Each job's output equals
 * its own lwl_bfht_linear_forward call bit for bit.  At decode batch sizes a
 * GPT-2 matrix has 18..72 generated blocks, so one matrix per launch leaves
 * most of the chip idle; jobs the bf16 matrix-core kernel takes with fewer
 * than 256 tokens run together, one launch per layer count for up to 48 jobs;
 * other jobs run as their single calls, so jobs do not run in job order.  All
 * jobs share `dtype`; outputs must not overlap, and no job's output may overlap
 * another job's input, latent, base or bias (the check rejects both); inputs
 * and latents may be shared.  A job's `epilogue` (NULL:
 * none) is that of lwl_bfht_linear_forward_ex; jobs whose epilogue has only a
 * bias still run grouped, jobs with a base or a row-sum term as single calls.
 * Workspace (query with the same jobs): the grouped jobs' own workspaces side
 * by side, plus the largest workspace of the jobs that run as single calls
 * (those run one after another on the stream and share it).
 */
typedef struct lwl_bfht_linear_job {
  const void* input;  /* [tokens, in_features] */
  const void* latent; /* [latent_size] */
  void* out;          /* [tokens, out_features] */
  int64_t tokens;
  int64_t in_features;
  int64_t latent_size;
  int64_t out_features;
  int64_t layers;
  int64_t seed;
  double weight_scale;
  const lwl_bfht_linear_epilogue* epilogue; /* or NULL */
} lwl_bfht_linear_job;

/* Host-only check of `count` jobs (each as lwl_bfht_check_linear_forward, plus disjoint outputs
 * and no output overlapping another job's operands). */
int lwl_bfht_check_linear_jobs(int dtype, const lwl_bfht_linear_job* jobs, int64_t count);
size_t lwl_bfht_linear_forward_grouped_workspace_size(int dtype, const lwl_bfht_linear_job* jobs, int64_t count);
int lwl_bfht_linear_forward_grouped(int dtype, const lwl_bfht_linear_job* jobs, int64_t count, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- fused latent gradient
 * Replaces the grad_latent branch of _BlockFHTLinearFn.backward (reference
 * latent_weight_lab/block_fht.py:339-352: grad_weight = grad^T @ input formed
 * in HBM, then block_fht_grad_latent; the reference's native extension has no
 * counterpart).
 *
 * grad_latent[p] = weight_scale * sum_b (D_0 H D_1 ... H D_L gw_b)[p], p < n,
 * with gw_b = (grad_out^T @ input) flattened, positions b*B .. b*B + B - 1:
 * the value lwl_bfht_backward gives for weight_scale * grad_weight, in one
 * call.  grad_out [tokens, out_features], input [tokens, in_features],
 * grad_latent [n], all bfloat16 (latent length 16385..32768: block 2^15), any
 * feature counts (rows off the 16-byte grid take element loads).  grad_weight
 * is formed by a split-K matrix-core GEMM as float32 partial sums over token
 * ranges in the workspace, summed in a fixed order, scaled and rounded once to
 * bf16 (the reference's grad_weight is bf16), then transformed by the
 * generator's backward; deterministic.  The modulation term of the reference
 * (block_fht.py:351-352) is left to the caller.  Workspace: query
 * *_workspace_size with the same shape (at config 4: 3 float32 partials of
 * in * out, a bf16 copy, the block rows).
 */
size_t lwl_bfht_linear_backward_latent_workspace_size(int64_t tokens, int64_t in_features,
                                                      int64_t out_features, int64_t latent_size);
int lwl_bfht_linear_backward_latent(const void* grad_out, const void* input, int dtype, int64_t tokens,
                                    int64_t in_features, int64_t latent_size, int64_t out_features,
                                    int64_t layers, int64_t seed, double weight_scale, void* grad_latent,
                                    void* workspace, size_t workspace_bytes, void* stream);

/* Host-only argument check of lwl_bfht_linear_backward_latent (no GPU needed). */
int lwl_bfht_check_linear_backward_latent(int dtype, int64_t tokens, int64_t in_features,
                                          int64_t latent_size, int64_t out_features, int64_t layers);

/* ---------------------------------------------------------------- weight cache, grouped
 * Replaces the per-module loops of prepare_block_fht_weight_cache and
 * flush_block_fht_weight_cache (reference latent_weight_lab/block_fht.py:560-569
 * over materialize_weight_cache :503-512 and flush_weight_cache_to_latent_grad
 * :514-557, each one ext.forward / ext.backward call, csrc/block_fht_ext_cuda.cu:516-622):
 * every job is one module's generator over the whole weight [0, size), and all
 * jobs run in a few launches.  T is the latent dtype, W the weight dtype:
 *
 *   materialize  weight[i] = W(T(T(y[i]) * weight_scale))
 *                (torch: (generator() * weight_scale).to(W))
 *   flush        r = T(T(adjoint(T(grad_weight))) * weight_scale)
 *                grad_latent = accumulate ? T(grad_latent + r) : r
 *                (torch: weight_scale * block_fht_grad_latent(latent,
 *                 grad_weight.to(T)), then latent.grad.add_ or assignment)
 *
 * Each block runs the code of the per-module call, so the results are
 * bit-identical to it.  Jobs take latents of length <= 32768 (blocks up to
 * 2^15); bfloat16 latents of block 2^15 need W = bfloat16.  Destinations must
 * not overlap.  Gains, modulation and residual weights stay with the caller.
 * The flush workspace holds every job's per-block partial rows (float32, or
 * bfloat16 for bfloat16 latents of block 2^15, as in the per-module call).
 */
typedef struct lwl_bfht_weight_job {
  const void* latent;      /* [latent_size], latent_dtype (materialize) */
  void* weight;            /* [size], weight_dtype (materialize: written) */
  const void* grad_weight; /* [size], weight_dtype (flush: read) */
  void* grad_latent;       /* [latent_size], latent_dtype (flush: written, read when accumulate) */
  int64_t latent_size;
  int64_t size;            /* in_features * out_features */
  int64_t layers;
  int64_t seed;
  int32_t latent_dtype;
  int32_t weight_dtype;
  double weight_scale;
  int32_t accumulate;      /* flush: add into grad_latent instead of overwriting it */
} lwl_bfht_weight_job;

/* Host-only check of count jobs for materialize (forward != 0) or flush. */
int lwl_bfht_check_weight_jobs(const lwl_bfht_weight_job* jobs, int64_t count, int forward);
int lwl_bfht_materialize_weights(const lwl_bfht_weight_job* jobs, int64_t count, void* stream);
size_t lwl_bfht_flush_weight_grads_workspace_size(const lwl_bfht_weight_job* jobs, int64_t count);
int lwl_bfht_flush_weight_grads(const lwl_bfht_weight_job* jobs, int64_t count, void* workspace,
                                size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- signed activation FHT
 * Replaces FixedFHTMix.forward (reference examples/nanogpt/model.py:200-218,
 * normalized_fht_last_dim :180-197), a torch loop of log2(P) reshape/clone
 * stages.  For each of `rows` rows of `features` values (row-major, contiguous):
 *
 *   out[row] = (S H S pad(x[row]))[:features]
 *
 * P = next power of two >= features (<= 32768), pad appends zeros, S =
 * diag(signs) with signs[P] = ±1.0f (the module's buffer, on the device), H the
 * Sylvester Walsh-Hadamard transform divided by sqrt(P).  float32 arithmetic,
 * one rounding to `dtype` at the end; float16 / bfloat16 rows of P = 1024 or
 * 4096 run on the matrix cores instead (operands in `dtype`, float32
 * accumulation: the intermediate of the two radix-32 stages is rounded once to
 * `dtype`, then the output once more).  S H S is symmetric, so the backward is
 * the same call on the output gradient.  out may equal x (in place).
 */
int lwl_fht_mix(const void* x, int dtype, int64_t rows, int64_t features, const float* signs, void* out,
                void* stream);
/* Host-only argument check of lwl_fht_mix. */
int lwl_fht_check_mix(int dtype, int64_t rows, int64_t features);

/* ---------------------------------------------------------------- sign words
 * Parity probe for the device hash (reference device functions
 * csrc/block_fht_ext_cuda.cu:27-43; Python twin block_fht.py:36-52):
 * out[i] = sign_word(seed, block, layer, first_word + i), computed on the GPU
 * by the same inlined code the transform kernels use.  out: nwords uint32.
 */
int lwl_bfht_sign_words(int64_t seed, int64_t block, int64_t layer, int64_t first_word,
                        int64_t nwords, uint32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LWL_BFHT_H */
