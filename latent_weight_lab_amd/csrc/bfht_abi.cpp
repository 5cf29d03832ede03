// C ABI of liblwl_bfht.so (declared in include/lwl_bfht.h).
//
// Host-side only: argument validation with the reference's messages, the
// execution plan (which kernels, how many overlapped blocks, workspace
// layout), and translation of HIP errors.  No device memory is allocated here.
#include "../../include/lwl_bfht.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <string>
#include <vector>

#include "bfht_launch.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return LWL_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(LWL_ERR_HIP, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

int log2_pow2_ceil(int64_t v) {
  int l = 0;
  while (((int64_t)1 << l) < v) ++l;
  return l;
}

uint32_t fold_seed(int64_t seed) {
  const uint64_t s = (uint64_t)seed;
  return (uint32_t)s ^ (uint32_t)(s >> 32);
}

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool valid_dtype(int d) { return d == LWL_DTYPE_F32 || d == LWL_DTYPE_F16 || d == LWL_DTYPE_BF16; }

// Checks shared by forward and backward.  Messages follow the reference:
// block_fht.py:13-14,92-93,609-610 and block_fht_ext_cuda.cu:524-529.
int check_common(int dtype, int64_t latent_size, int64_t output_size, int64_t layers,
                 int64_t start, int64_t stop) {
  if (!valid_dtype(dtype))
    return fail(LWL_ERR_UNSUPPORTED, "Block-FHT supports float32, float16 and bfloat16 (dtype code %d)",
                dtype);
  if (latent_size <= 0) return fail(LWL_ERR_INVALID, "latent size must be positive");
  if (output_size <= 0) return fail(LWL_ERR_INVALID, "size must be positive");
  if (layers < 1 || layers > 3) return fail(LWL_ERR_INVALID, "layers must be 1, 2, or 3");
  if (!(0 <= start && start <= stop && stop <= output_size))
    return fail(LWL_ERR_INVALID, "invalid slice [%lld, %lld) for size %lld", (long long)start,
                (long long)stop, (long long)output_size);
  if (latent_size > LWL_BFHT_MAX_BLOCK_SIZE)
    return fail(LWL_ERR_UNSUPPORTED,
                "Block-FHT supports power-of-two block sizes up to 2^23 after padding (latent size %lld)",
                (long long)latent_size);
  return LWL_OK;
}

lwl::BfhtArgs plan(int dtype, int64_t latent_size, int64_t layers, int64_t seed, int64_t start,
                   int64_t stop) {
  lwl::BfhtArgs a{};
  a.dtype = dtype;
  a.n = latent_size;
  a.log_block = log2_pow2_ceil(latent_size);
  const int64_t B = (int64_t)1 << a.log_block;
  a.first_block = start / B;
  a.nblocks = stop > start ? (stop + B - 1) / B - a.first_block : 0;
  a.start = start;
  a.stop = stop;
  a.seed32 = fold_seed(seed);
  a.layers = (int)layers;
  return a;
}

size_t forward_ws(const lwl::BfhtArgs& a) {
  // the tile passes' float32 work buffer, for one group of blocks at a time
  if (a.log_block <= lwl::kWholeBlockMaxLog || a.nblocks == 0) return 0;
  const int64_t blocks = std::min<int64_t>(a.nblocks, lwl::tile_group_blocks(a.log_block));
  return align_up((size_t)blocks * ((size_t)1 << a.log_block) * sizeof(float));
}

size_t backward_ws(const lwl::BfhtArgs& a) {
  if (a.nblocks == 0) return 0;
  // whole-block kernels: one float32 partial row of n values per block, or
  // (matrix-core kernel, which writes it even for a single block) one
  // bfloat16 row padded to 8 values
  if (a.log_block <= lwl::kWholeBlockMaxLog) {
    const size_t row = std::max((size_t)a.n * sizeof(float), (size_t)lwl::mfma15_part_stride(a.n) * 2);
    return align_up((size_t)a.nblocks * row);
  }
  return align_up((size_t)a.nblocks * ((size_t)1 << a.log_block) * sizeof(float));
}

// Fused linear checks; messages follow block_fht_ext_cuda.cu:631-644 and
// block_fht.py:259-260.  Two kernels share the entry point: the matrix-core one
// (bf16, block 2^15; any in_features in its range, rows may straddle blocks)
// and the reference extension's own domain (float32 / float16 / bfloat16,
// block <= 2^14, block % in_features == 0).  Sizes that would overflow their
// 32-bit buffer offsets or grid dimensions are rejected as unsupported (the
// caller then generates W and calls a GEMM).
int check_linear(int dtype, int64_t tokens, int64_t in_features, int64_t latent_size,
                 int64_t out_features, int64_t layers) {
  if (!valid_dtype(dtype))
    return fail(LWL_ERR_UNSUPPORTED,
                "fused linear forward supports float32, float16, and bfloat16 (dtype code %d)", dtype);
  if (tokens < 0) return fail(LWL_ERR_INVALID, "tokens must be non-negative");
  if (in_features <= 0) return fail(LWL_ERR_INVALID, "in_features must be positive");
  if (out_features <= 0) return fail(LWL_ERR_INVALID, "out_features must be positive");
  if (layers < 1 || layers > 3) return fail(LWL_ERR_INVALID, "layers must be 1, 2, or 3");
  if (latent_size <= 0) return fail(LWL_ERR_INVALID, "latent size must be positive");
  const int lb = log2_pow2_ceil(latent_size);
  if (lb > lwl::kWholeBlockMaxLog)
    return fail(LWL_ERR_UNSUPPORTED,
                "fused linear forward supports block sizes up to 2^15 (latent size %lld)",
                (long long)latent_size);
  if (in_features > ((int64_t)1 << lb))
    return fail(LWL_ERR_UNSUPPORTED, "fused linear forward requires in_features <= block_size");
  const int64_t esize = dtype == LWL_DTYPE_F32 ? 4 : 2;
  const int64_t kOffsetLimit = (int64_t)1 << 31;
  if (lwl::kLinearKernelAvailable && lwl::linear_applicable(dtype, lb, in_features)) {
    if (tokens * in_features * 2 >= kOffsetLimit)
      return fail(LWL_ERR_UNSUPPORTED, "fused linear forward: tokens * in_features must stay below 2^30");
    // the epilogue addresses 16 tokens' rows of out from one buffer resource
    if (out_features * 16 * 2 >= kOffsetLimit)
      return fail(LWL_ERR_UNSUPPORTED, "fused linear forward: out_features must stay below 2^26");
    // the straddling-row combine runs one grid row per tile boundary
    const int64_t nblocks = (in_features * out_features + ((int64_t)1 << lb) - 1) >> lb;
    if (nblocks > 65536)
      return fail(LWL_ERR_UNSUPPORTED, "fused linear forward: in_features * out_features must stay below 2^31");
    return LWL_OK;
  }
  if (lwl::linear_small_applicable(dtype, lb, in_features)) {
    if (tokens * in_features * esize >= kOffsetLimit || tokens * out_features * esize >= kOffsetLimit)
      return fail(LWL_ERR_UNSUPPORTED,
                  "fused linear forward: tokens * in_features and tokens * out_features must stay below 2 GiB");
    return LWL_OK;
  }
  return fail(LWL_ERR_UNSUPPORTED,
              "fused linear forward takes (a) bfloat16 latents of length 16385..32768 (block 2^15) with "
              "in_features %% 8 == 0 and 528 <= in_features <= 5120, or (b) float32, float16 or bfloat16 "
              "latents of block <= 2^14 with block_size %% in_features == 0 (dtype code %d, latent size %lld, "
              "in_features %lld)",
              dtype, (long long)latent_size, (long long)in_features);
}

bool linear_uses_mfma(const lwl::LinearArgs& a) {
  return lwl::linear_applicable(a.dtype, a.log_block, a.in_features);
}

lwl::LinearArgs plan_linear(int dtype, int64_t tokens, int64_t in_features, int64_t latent_size,
                            int64_t out_features, int64_t layers, int64_t seed,
                            double weight_scale) {
  lwl::LinearArgs a{};
  a.dtype = dtype;
  a.tokens = tokens;
  a.in_features = in_features;
  a.out_features = out_features;
  a.n = latent_size;
  a.log_block = log2_pow2_ceil(latent_size);
  const int64_t B = (int64_t)1 << a.log_block;
  a.nblocks_w = (in_features * out_features + B - 1) / B;
  a.seed32 = fold_seed(seed);
  a.layers = (int)layers;
  a.weight_scale = (float)weight_scale;
  a.blocks_per_wg = 1;
  if (linear_uses_mfma(a)) {
    a.blocks_per_wg = lwl::linear_blocks_per_wg(a);
    a.rows_per_tile = lwl::linear_rows_per_tile(a);
    a.token_splits = lwl::linear_token_splits(a);
  } else if (lwl::linear_small_mm_applicable(a)) {
    a.token_splits = lwl::linear_small_mm_token_splits(a);
  } else {
    a.token_splits = lwl::linear_small_token_splits(a);
  }
  return a;
}

// Workspace: the block-2^15 kernel's partial rows and tiled x; in the
// reference's domain the tiled x of the matrix-core kernel (256 tokens and
// more), else none.
size_t linear_ws(const lwl::LinearArgs& a) {
  return align_up(linear_uses_mfma(a) ? lwl::linear_workspace_bytes(a) : lwl::linear_small_mm_workspace_bytes(a));
}

// Epilogue (lwl_bfht_linear_forward_ex): the kernels' form of it, and the
// workspace it adds after linear_ws (float32 row sums of x, with a row-sum term).
lwl::LinearEpi epilogue_of(const lwl_bfht_linear_epilogue* ep) {
  lwl::LinearEpi e{};
  if (!ep) return e;
  e.bias = ep->bias;
  e.base = ep->base;
  e.coef = ep->row_sum_coef;
  e.cscale = (float)ep->row_sum_scale;
  return e;
}
size_t row_sum_ws(const lwl::LinearArgs& a) { return a.epi.coef ? align_up((size_t)a.tokens * sizeof(float)) : 0; }
size_t linear_ex_ws(const lwl::LinearArgs& a) { return linear_ws(a) + row_sum_ws(a); }

// Launches one fused linear (a.x, a.latent, a.out, a.epi set; a.work at least
// linear_ex_ws bytes): the row sums first when the epilogue has a row-sum term.
hipError_t launch_linear_ex(lwl::LinearArgs a, hipStream_t s) {
  if (a.epi.coef) {
    float* xsum = (float*)((unsigned char*)a.work + linear_ws(a));
    const hipError_t e = lwl::launch_row_sums(a, xsum, s);
    if (e != hipSuccess) return e;
    a.epi.xsum = xsum;
  }
  if (linear_uses_mfma(a)) return lwl::launch_linear(a, s);
  return lwl::linear_small_mm_applicable(a) ? lwl::launch_linear_small_mm(a, s) : lwl::launch_linear_small(a, s);
}

// Fused latent-gradient checks (no reference counterpart: the reference forms
// grad_weight in HBM, block_fht.py:339-352).
int check_linear_bwd(int dtype, int64_t tokens, int64_t in_features, int64_t latent_size, int64_t out_features,
                     int64_t layers) {
  if (!valid_dtype(dtype))
    return fail(LWL_ERR_UNSUPPORTED, "linear latent gradient supports float32, float16, and bfloat16 (dtype code %d)",
                dtype);
  if (tokens < 0) return fail(LWL_ERR_INVALID, "tokens must be non-negative");
  if (in_features <= 0) return fail(LWL_ERR_INVALID, "in_features must be positive");
  if (out_features <= 0) return fail(LWL_ERR_INVALID, "out_features must be positive");
  if (layers < 1 || layers > 3) return fail(LWL_ERR_INVALID, "layers must be 1, 2, or 3");
  if (latent_size <= 0) return fail(LWL_ERR_INVALID, "latent size must be positive");
  const int lb = log2_pow2_ceil(latent_size);
  if (lb > lwl::kWholeBlockMaxLog || !lwl::linear_bwd_applicable(dtype, lb, in_features))
    return fail(LWL_ERR_UNSUPPORTED,
                "fused linear latent gradient takes bfloat16 latents of length 16385..32768 (block 2^15) "
                "(dtype code %d, latent size %lld)",
                dtype, (long long)latent_size);
  // 32-bit buffer offsets: token-major operands, and each float32 partial of grad_weight
  if (tokens * in_features * 2 >= ((int64_t)1 << 31) || tokens * out_features * 2 >= ((int64_t)1 << 31))
    return fail(LWL_ERR_UNSUPPORTED,
                "fused linear latent gradient: tokens * in_features and tokens * out_features must stay below 2^30");
  if (in_features * out_features >= ((int64_t)1 << 29))
    return fail(LWL_ERR_UNSUPPORTED, "fused linear latent gradient: in_features * out_features must stay below 2^29");
  return LWL_OK;
}

lwl::LinearBwdArgs plan_linear_bwd(int64_t tokens, int64_t in_features, int64_t latent_size, int64_t out_features,
                                   int64_t layers, int64_t seed, double weight_scale) {
  lwl::LinearBwdArgs a{};
  a.tokens = tokens;
  a.in_features = in_features;
  a.out_features = out_features;
  a.n = latent_size;
  a.log_block = log2_pow2_ceil(latent_size);
  const int64_t B = (int64_t)1 << a.log_block;
  a.nblocks_w = (in_features * out_features + B - 1) / B;
  a.seed32 = fold_seed(seed);
  a.layers = (int)layers;
  a.weight_scale = (float)weight_scale;
  a.token_splits = lwl::linear_bwd_token_splits(a);
  return a;
}

// Grouped fused linear: every job checked as a single call; outputs disjoint.
int check_linear_jobs(int dtype, const lwl_bfht_linear_job* jobs, int64_t count, bool need_ptrs,
                      std::vector<lwl::LinearArgs>* out) {
  if (count < 0) return fail(LWL_ERR_INVALID, "job count must be non-negative");
  if (count > 0 && !jobs) return fail(LWL_ERR_INVALID, "jobs must be non-null");
  std::vector<lwl::LinearArgs> v((size_t)count);
  const int64_t esize = dtype == LWL_DTYPE_F32 ? 4 : 2;
  for (int64_t i = 0; i < count; ++i) {
    const lwl_bfht_linear_job& j = jobs[i];
    const int rc = check_linear(dtype, j.tokens, j.in_features, j.latent_size, j.out_features, j.layers);
    if (rc) return fail(rc, "job %lld: %s", (long long)i, g_last_error.c_str());
    if (need_ptrs && j.tokens > 0 && (!j.input || !j.latent || !j.out))
      return fail(LWL_ERR_INVALID, "job %lld: input, latent and out must be non-null", (long long)i);
    v[(size_t)i] = plan_linear(dtype, j.tokens, j.in_features, j.latent_size, j.out_features, j.layers, j.seed,
                               j.weight_scale);
    v[(size_t)i].x = j.input;
    v[(size_t)i].latent = j.latent;
    v[(size_t)i].out = j.out;
    v[(size_t)i].epi = epilogue_of(j.epilogue);
  }
  if (need_ptrs) {
    // [p, p + bytes) ranges; empty ranges and null pointers overlap nothing
    auto overlap = [](const void* p, int64_t bytes, const void* q, int64_t qbytes) {
      const uintptr_t x0 = (uintptr_t)p, y0 = (uintptr_t)q;
      return p && q && bytes > 0 && qbytes > 0 && x0 < y0 + (uintptr_t)qbytes && y0 < x0 + (uintptr_t)bytes;
    };
    for (int64_t a = 0; a < count; ++a) {
      const int64_t out_bytes = jobs[a].tokens * jobs[a].out_features * esize;
      for (int64_t b = 0; b < count; ++b) {
        const lwl_bfht_linear_job& jb = jobs[b];
        if (b > a && overlap(jobs[a].out, out_bytes, jb.out, jb.tokens * jb.out_features * esize))
          return fail(LWL_ERR_INVALID, "jobs %lld and %lld write overlapping outputs", (long long)a, (long long)b);
        // jobs do not run in job order (grouped ones share launches), so no job may
        // read what another job writes (a job's own operands follow its single call)
        if (b == a) continue;
        const lwl_bfht_linear_epilogue* e = jb.tokens > 0 ? jb.epilogue : nullptr;
        const char* what = overlap(jobs[a].out, out_bytes, jb.input, jb.tokens * jb.in_features * esize) ? "input"
                         : overlap(jobs[a].out, out_bytes, jb.latent, jb.tokens > 0 ? jb.latent_size * esize : 0)
                             ? "latent"
                         : (e && overlap(jobs[a].out, out_bytes, e->base, jb.tokens * jb.out_features * esize))
                             ? "base"
                         : (e && overlap(jobs[a].out, out_bytes, e->bias, jb.out_features * esize)) ? "bias"
                                                                                                    : nullptr;
        if (what)
          return fail(LWL_ERR_INVALID, "job %lld's output overlaps job %lld's %s", (long long)a, (long long)b, what);
      }
    }
  }
  if (out) *out = std::move(v);
  return LWL_OK;
}

int check_workspace(size_t need, const void* ws, size_t have) {
  if (need == 0) return LWL_OK;
  if (ws == nullptr || have < need)
    return fail(LWL_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need,
                ws ? have : (size_t)0);
  if ((uintptr_t)ws % kAlign) return fail(LWL_ERR_WORKSPACE, "workspace must be %zu-byte aligned", kAlign);
  return LWL_OK;
}

// Grouped weight-cache jobs (block_fht.py:503-569): each job is the whole
// weight of one module, with the per-module call's checks.
int check_weight_jobs(const lwl_bfht_weight_job* jobs, int64_t count, bool fwd, std::vector<lwl::WeightJob>* out) {
  if (count < 0) return fail(LWL_ERR_INVALID, "job count must be non-negative");
  if (count > 0 && !jobs) return fail(LWL_ERR_INVALID, "jobs must be non-null");
  std::vector<lwl::WeightJob> v((size_t)count);
  for (int64_t i = 0; i < count; ++i) {
    const lwl_bfht_weight_job& j = jobs[i];
    int rc = check_common(j.latent_dtype, j.latent_size, j.size, j.layers, 0, j.size);
    if (rc) return fail(rc, "job %lld: %s", (long long)i, g_last_error.c_str());
    if (!valid_dtype(j.weight_dtype))
      return fail(LWL_ERR_UNSUPPORTED, "job %lld: weight dtype code %d is not float32, float16 or bfloat16",
                  (long long)i, j.weight_dtype);
    if (fwd ? (!j.latent || !j.weight) : (!j.grad_weight || !j.grad_latent))
      return fail(LWL_ERR_INVALID, "job %lld: %s must be non-null", (long long)i,
                  fwd ? "latent and weight" : "grad_weight and grad_latent");
    lwl::WeightJob w{};
    w.latent = j.latent;
    w.weight = j.weight;
    w.grad_weight = j.grad_weight;
    w.grad_latent = j.grad_latent;
    w.n = j.latent_size;
    w.size = j.size;
    w.layers = (int)j.layers;
    w.seed32 = fold_seed(j.seed);
    w.ldtype = j.latent_dtype;
    w.wdtype = j.weight_dtype;
    w.scale = (float)j.weight_scale;
    w.accumulate = j.accumulate != 0;
    const char* why = nullptr;
    if (!lwl::grouped_job_supported(w, fwd, &why)) return fail(LWL_ERR_UNSUPPORTED, "job %lld: %s", (long long)i, why);
    v[(size_t)i] = w;
  }
  // destinations pairwise disjoint (one launch writes them all)
  auto esize = [](int d) { return d == LWL_DTYPE_F32 ? 4 : 2; };
  for (int64_t a = 0; a < count; ++a)
    for (int64_t b = a + 1; b < count; ++b) {
      const auto& x = v[(size_t)a];
      const auto& y = v[(size_t)b];
      const uintptr_t x0 = (uintptr_t)(fwd ? x.weight : x.grad_latent);
      const uintptr_t y0 = (uintptr_t)(fwd ? y.weight : y.grad_latent);
      const uintptr_t x1 = x0 + (uintptr_t)(fwd ? x.size * esize(x.wdtype) : x.n * esize(x.ldtype));
      const uintptr_t y1 = y0 + (uintptr_t)(fwd ? y.size * esize(y.wdtype) : y.n * esize(y.ldtype));
      if (x0 < y1 && y0 < x1)
        return fail(LWL_ERR_INVALID, "jobs %lld and %lld write overlapping memory", (long long)a, (long long)b);
    }
  if (out) *out = std::move(v);
  return LWL_OK;
}

}  // namespace

extern "C" {

const char* lwl_last_error(void) { return g_last_error.c_str(); }

int lwl_abi_version(void) { return 2; }

int lwl_bfht_check_forward(int dtype, int64_t latent_size, int64_t output_size, int64_t layers,
                           int64_t start, int64_t stop) {
  const int rc = check_common(dtype, latent_size, output_size, layers, start, stop);
  return rc ? rc : ok();
}

size_t lwl_bfht_forward_workspace_size(int64_t latent_size, int64_t output_size, int64_t start,
                                       int64_t stop) {
  if (check_common(LWL_DTYPE_F32, latent_size, output_size, 1, start, stop)) return 0;
  return forward_ws(plan(LWL_DTYPE_F32, latent_size, 1, 0, start, stop));
}

int lwl_bfht_forward(const void* latent, int dtype, int64_t latent_size, int64_t output_size,
                     int64_t layers, int64_t seed, int64_t start, int64_t stop, void* out,
                     void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_common(dtype, latent_size, output_size, layers, start, stop);
  if (rc) return rc;
  lwl::BfhtArgs a = plan(dtype, latent_size, layers, seed, start, stop);
  if (a.nblocks == 0) return ok();
  if (!latent || !out) return fail(LWL_ERR_INVALID, "latent and out must be non-null");
  rc = check_workspace(forward_ws(a), workspace, workspace_bytes);
  if (rc) return rc;
  a.src = latent;
  a.dst = out;
  a.work = workspace;
  return hip_status(lwl::launch_bfht(a, (hipStream_t)stream, true), "lwl_bfht_forward");
}

size_t lwl_bfht_backward_workspace_size(int64_t latent_size, int64_t output_size, int64_t start,
                                        int64_t stop) {
  if (check_common(LWL_DTYPE_F32, latent_size, output_size, 1, start, stop)) return 0;
  return backward_ws(plan(LWL_DTYPE_F32, latent_size, 1, 0, start, stop));
}

int lwl_bfht_backward(const void* grad_out, int dtype, int64_t latent_size, int64_t output_size,
                      int64_t layers, int64_t seed, int64_t start, int64_t stop, void* grad_latent,
                      void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_common(dtype, latent_size, output_size, layers, start, stop);
  if (rc) return rc;
  lwl::BfhtArgs a = plan(dtype, latent_size, layers, seed, start, stop);
  if (!grad_latent || (a.nblocks > 0 && !grad_out))
    return fail(LWL_ERR_INVALID, "grad_out and grad_latent must be non-null");
  rc = check_workspace(backward_ws(a), workspace, workspace_bytes);
  if (rc) return rc;
  a.src = grad_out;
  a.dst = grad_latent;
  a.work = workspace;
  return hip_status(lwl::launch_bfht(a, (hipStream_t)stream, false), "lwl_bfht_backward");
}

int lwl_bfht_backward_noalloc(const void* grad_out, int dtype, int64_t latent_size, int64_t output_size,
                              int64_t layers, int64_t seed, int64_t start, int64_t stop, void* grad_latent,
                              void* stream) {
  int rc = check_common(dtype, latent_size, output_size, layers, start, stop);
  if (rc) return rc;
  lwl::BfhtArgs a = plan(dtype, latent_size, layers, seed, start, stop);
  if (!grad_latent || (a.nblocks > 0 && !grad_out))
    return fail(LWL_ERR_INVALID, "grad_out and grad_latent must be non-null");
  const size_t need = backward_ws(a);
  if (need > (size_t)LWL_BFHT_NOALLOC_SCRATCH_BYTES)
    return fail(LWL_ERR_UNSUPPORTED,
                "lwl_bfht_backward_noalloc: this call needs %zu bytes of scratch, more than the %zu of its "
                "device array; call lwl_bfht_backward with a workspace",
                need, (size_t)LWL_BFHT_NOALLOC_SCRATCH_BYTES);
  // every accepted call resolves the device's array address (the first one per
  // device asks hipGetSymbolAddress; later ones read the cached address), even
  // one that needs no scratch, so a caller can settle it before a graph capture
  hipError_t e = hipSuccess;
  void* scratch = lwl::noalloc_scratch((hipStream_t)stream, &e);
  if (!scratch) return hip_status(e, "lwl_bfht_backward_noalloc: scratch address");
  void* work = need > 0 ? scratch : nullptr;
  a.src = grad_out;
  a.dst = grad_latent;
  a.work = work;
  return hip_status(lwl::launch_bfht(a, (hipStream_t)stream, false), "lwl_bfht_backward_noalloc");
}

int lwl_bfht_check_linear_forward(int dtype, int64_t tokens, int64_t in_features,
                                  int64_t latent_size, int64_t out_features, int64_t layers) {
  const int rc = check_linear(dtype, tokens, in_features, latent_size, out_features, layers);
  return rc ? rc : ok();
}

size_t lwl_bfht_linear_forward_workspace_size(int64_t tokens, int64_t in_features,
                                              int64_t out_features, int64_t latent_size) {
  // The query has no dtype (as ext.linear_forward has none): it returns the
  // most any dtype needs for the shape (float32 in the reference's domain, whose
  // tiled x copy is twice the 16-bit one), 0 where no fused kernel takes it.
  size_t most = 0;
  for (int dtype : {LWL_DTYPE_F32, LWL_DTYPE_F16, LWL_DTYPE_BF16})
    if (!check_linear(dtype, tokens, in_features, latent_size, out_features, 1))
      most = std::max(most, linear_ws(plan_linear(dtype, tokens, in_features, latent_size, out_features, 1, 0, 1.0)));
  return most;
}

int lwl_bfht_linear_forward(const void* input, const void* latent, int dtype, int64_t tokens,
                            int64_t in_features, int64_t latent_size, int64_t out_features,
                            int64_t layers, int64_t seed, double weight_scale, void* out,
                            void* workspace, size_t workspace_bytes, void* stream) {
  return lwl_bfht_linear_forward_ex(input, latent, dtype, tokens, in_features, latent_size, out_features, layers,
                                    seed, weight_scale, nullptr, out, workspace, workspace_bytes, stream);
}

size_t lwl_bfht_linear_forward_ex_workspace_size(int dtype, int64_t tokens, int64_t in_features,
                                                 int64_t out_features, int64_t latent_size,
                                                 const lwl_bfht_linear_epilogue* epilogue) {
  if (check_linear(dtype, tokens, in_features, latent_size, out_features, 1)) return 0;
  lwl::LinearArgs a = plan_linear(dtype, tokens, in_features, latent_size, out_features, 1, 0, 1.0);
  a.epi = epilogue_of(epilogue);
  return linear_ex_ws(a);
}

int lwl_bfht_linear_forward_ex(const void* input, const void* latent, int dtype, int64_t tokens,
                               int64_t in_features, int64_t latent_size, int64_t out_features,
                               int64_t layers, int64_t seed, double weight_scale,
                               const lwl_bfht_linear_epilogue* epilogue, void* out, void* workspace,
                               size_t workspace_bytes, void* stream) {
  int rc = check_linear(dtype, tokens, in_features, latent_size, out_features, layers);
  if (rc) return rc;
  if (tokens == 0) return ok();
  if (!input || !latent || !out)
    return fail(LWL_ERR_INVALID, "input, latent and out must be non-null");
  lwl::LinearArgs a = plan_linear(dtype, tokens, in_features, latent_size, out_features, layers,
                                  seed, weight_scale);
  a.epi = epilogue_of(epilogue);
  rc = check_workspace(linear_ex_ws(a), workspace, workspace_bytes);
  if (rc) return rc;
  a.x = input;
  a.latent = latent;
  a.out = out;
  a.work = workspace;
  return hip_status(launch_linear_ex(a, (hipStream_t)stream), "lwl_bfht_linear_forward");
}

int lwl_bfht_check_linear_jobs(int dtype, const lwl_bfht_linear_job* jobs, int64_t count) {
  const int rc = check_linear_jobs(dtype, jobs, count, true, nullptr);
  return rc ? rc : ok();
}

// Grouped workspace: the grouped jobs' partial rows side by side (one launch
// reads them all), then one region that the jobs running as single launches
// reuse one after another (the largest of their workspaces).
// Grouped: the matrix-core kernel's jobs below its tiled-x batch whose epilogue
// is at most a bias (the grouped table carries one bias pointer per job).
bool job_grouped(const lwl::LinearArgs& a) {
  return a.tokens > 0 && linear_uses_mfma(a) && lwl::linear_groupable(a) && !a.epi.base && !a.epi.coef;
}

size_t grouped_ws(const std::vector<lwl::LinearArgs>& v) {
  size_t together = 0, single = 0;
  for (const auto& a : v) {
    if (a.tokens == 0) continue;
    if (job_grouped(a)) together += linear_ws(a);
    else single = std::max(single, linear_ex_ws(a));
  }
  return together + single;
}

size_t lwl_bfht_linear_forward_grouped_workspace_size(int dtype, const lwl_bfht_linear_job* jobs, int64_t count) {
  std::vector<lwl::LinearArgs> v;
  if (check_linear_jobs(dtype, jobs, count, false, &v)) return 0;
  return grouped_ws(v);
}

int lwl_bfht_linear_forward_grouped(int dtype, const lwl_bfht_linear_job* jobs, int64_t count, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  std::vector<lwl::LinearArgs> v;
  int rc = check_linear_jobs(dtype, jobs, count, true, &v);
  if (rc) return rc;
  rc = check_workspace(grouped_ws(v), workspace, workspace_bytes);
  if (rc) return rc;
  // grouped jobs: their own partial-row slices (256-byte multiples, in job
  // order); the others: one shared region after them, used in turn on the stream
  std::vector<lwl::LinearArgs> grouped;
  size_t off = 0;
  for (auto& a : v)
    if (job_grouped(a)) {
      a.work = (unsigned char*)workspace + off;
      off += linear_ws(a);
      grouped.push_back(a);
    }
  for (auto& a : v) {
    if (a.tokens == 0 || job_grouped(a)) continue;
    a.work = linear_ex_ws(a) ? (unsigned char*)workspace + off : nullptr;
    const hipError_t e = launch_linear_ex(a, (hipStream_t)stream);
    if (e != hipSuccess) return hip_status(e, "lwl_bfht_linear_forward_grouped");
  }
  return hip_status(lwl::launch_linear_grouped(grouped.data(), (int64_t)grouped.size(), (hipStream_t)stream),
                    "lwl_bfht_linear_forward_grouped");
}

int lwl_bfht_check_linear_backward_latent(int dtype, int64_t tokens, int64_t in_features,
                                          int64_t latent_size, int64_t out_features, int64_t layers) {
  const int rc = check_linear_bwd(dtype, tokens, in_features, latent_size, out_features, layers);
  return rc ? rc : ok();
}

size_t lwl_bfht_linear_backward_latent_workspace_size(int64_t tokens, int64_t in_features,
                                                      int64_t out_features, int64_t latent_size) {
  if (check_linear_bwd(LWL_DTYPE_BF16, tokens, in_features, latent_size, out_features, 1)) return 0;
  if (tokens == 0) return 0;
  return align_up(lwl::linear_bwd_workspace_bytes(
      plan_linear_bwd(tokens, in_features, latent_size, out_features, 1, 0, 1.0)));
}

int lwl_bfht_linear_backward_latent(const void* grad_out, const void* input, int dtype, int64_t tokens,
                                    int64_t in_features, int64_t latent_size, int64_t out_features,
                                    int64_t layers, int64_t seed, double weight_scale, void* grad_latent,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_linear_bwd(dtype, tokens, in_features, latent_size, out_features, layers);
  if (rc) return rc;
  if (!grad_latent) return fail(LWL_ERR_INVALID, "grad_latent must be non-null");
  if (tokens > 0 && (!grad_out || !input)) return fail(LWL_ERR_INVALID, "grad_out and input must be non-null");
  lwl::LinearBwdArgs a = plan_linear_bwd(tokens, in_features, latent_size, out_features, layers, seed, weight_scale);
  if (tokens == 0) {
    // no tokens: the gradient is zero (a block sum over zero partial rows)
    return hip_status(lwl::launch_block_sum(nullptr, 0, latent_size, latent_size, grad_latent, dtype,
                                            (hipStream_t)stream),
                      "lwl_bfht_linear_backward_latent");
  }
  rc = check_workspace(lwl::linear_bwd_workspace_bytes(a), workspace, workspace_bytes);
  if (rc) return rc;
  a.grad = grad_out;
  a.x = input;
  a.grad_latent = grad_latent;
  a.work = workspace;
  return hip_status(lwl::launch_linear_bwd(a, (hipStream_t)stream), "lwl_bfht_linear_backward_latent");
}

int lwl_bfht_check_weight_jobs(const lwl_bfht_weight_job* jobs, int64_t count, int forward) {
  const int rc = check_weight_jobs(jobs, count, forward != 0, nullptr);
  return rc ? rc : ok();
}

int lwl_bfht_materialize_weights(const lwl_bfht_weight_job* jobs, int64_t count, void* stream) {
  std::vector<lwl::WeightJob> v;
  const int rc = check_weight_jobs(jobs, count, true, &v);
  if (rc) return rc;
  return hip_status(lwl::launch_grouped(v.data(), count, nullptr, (hipStream_t)stream, true),
                    "lwl_bfht_materialize_weights");
}

size_t lwl_bfht_flush_weight_grads_workspace_size(const lwl_bfht_weight_job* jobs, int64_t count) {
  std::vector<lwl::WeightJob> v;
  if (check_weight_jobs(jobs, count, false, &v)) return 0;
  return lwl::grouped_workspace_bytes(v.data(), count);
}

int lwl_bfht_flush_weight_grads(const lwl_bfht_weight_job* jobs, int64_t count, void* workspace,
                                size_t workspace_bytes, void* stream) {
  std::vector<lwl::WeightJob> v;
  int rc = check_weight_jobs(jobs, count, false, &v);
  if (rc) return rc;
  rc = check_workspace(lwl::grouped_workspace_bytes(v.data(), count), workspace, workspace_bytes);
  if (rc) return rc;
  return hip_status(lwl::launch_grouped(v.data(), count, workspace, (hipStream_t)stream, false),
                    "lwl_bfht_flush_weight_grads");
}

int lwl_fht_check_mix(int dtype, int64_t rows, int64_t features) {
  if (!valid_dtype(dtype))
    return fail(LWL_ERR_UNSUPPORTED, "FHT mix supports float32, float16 and bfloat16 (dtype code %d)", dtype);
  if (rows < 0) return fail(LWL_ERR_INVALID, "rows must be non-negative");
  if (features <= 0) return fail(LWL_ERR_INVALID, "features must be positive");
  if (features > ((int64_t)1 << lwl::kWholeBlockMaxLog))
    return fail(LWL_ERR_UNSUPPORTED, "FHT mix supports up to 32768 features (got %lld)", (long long)features);
  if (rows > ((int64_t)1 << 40)) return fail(LWL_ERR_UNSUPPORTED, "too many rows");
  return ok();
}

int lwl_fht_mix(const void* x, int dtype, int64_t rows, int64_t features, const float* signs, void* out,
                void* stream) {
  const int rc = lwl_fht_check_mix(dtype, rows, features);
  if (rc) return rc;
  if (rows == 0) return ok();
  if (!x || !signs || !out) return fail(LWL_ERR_INVALID, "x, signs and out must be non-null");
  return hip_status(lwl::launch_fht_mix(dtype, x, out, signs, rows, features, log2_pow2_ceil(features),
                                        (hipStream_t)stream),
                    "lwl_fht_mix");
}

int lwl_bfht_sign_words(int64_t seed, int64_t block, int64_t layer, int64_t first_word,
                        int64_t nwords, uint32_t* out, void* stream) {
  if (nwords < 0 || first_word < 0 || (nwords > 0 && !out))
    return fail(LWL_ERR_INVALID, "invalid sign-word request");
  if (first_word + nwords > ((int64_t)1 << 32))
    return fail(LWL_ERR_INVALID, "word index exceeds 32 bits");
  return hip_status(lwl::launch_sign_words(fold_seed(seed), block, (int)layer, first_word, nwords,
                                           out, (hipStream_t)stream),
                    "lwl_bfht_sign_words");
}

}  // extern "C"
