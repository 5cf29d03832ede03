// Planner of the grouped weight-cache calls: many generators (one per
// BlockFHTLinear module) materialized, or their weight gradients projected back
// onto the latents, in a few launches instead of one or two per module.
//
// Reference: latent_weight_lab/block_fht.py:503-569 (materialize_weight_cache,
// flush_weight_cache_to_latent_grad and the model-wide prepare / flush loops,
// one ext.forward / ext.backward call per module).  Jobs are sorted into
// classes that one kernel instantiation serves — (matrix-core chain, layer
// count) for bfloat16 blocks of 2^15 that the per-module call would run on the
// matrix cores, (latent type, weight type, block size) for every other whole
// block — and
// each class runs in launches of up to kGroupMaxJobs jobs.  Every block runs
// exactly the code of its per-module launch, so the results are bit-identical
// to the per-module path followed by torch's scale, cast and accumulate.
#include <hip/hip_runtime_api.h>

#include <vector>

#include "bfht_launch.h"

namespace lwl {
namespace {

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

int log2_ceil(int64_t v) {
  int l = 0;
  while (((int64_t)1 << l) < v) ++l;
  return l;
}

struct ClassKey {
  bool mfma;
  int dtype;
  int wdtype;  // VALU classes only (a template parameter there)
  int log_block;
  int layers;  // matrix-core classes only (a template parameter there)
  bool operator==(const ClassKey& o) const {
    return mfma == o.mfma && dtype == o.dtype && wdtype == o.wdtype && log_block == o.log_block &&
           layers == o.layers;
  }
};

ClassKey class_of(const WeightJob& j, bool fwd) {
  const int lb = log2_ceil(j.n);
  // the per-module matrix-core predicate (mfma15_applicable): bf16, block 2^15,
  // a 16-byte aligned source (latent, or the weight gradient in the backward);
  // a bf16 weight gradient at any 2-byte offset too (the kernel reads aligned
  // 16-byte slots), as in the per-module backward
  const void* src = fwd ? j.latent : j.grad_weight;
  const bool aligned = (uintptr_t)src % 16 == 0 || (!fwd && j.wdtype == kBF16 && (uintptr_t)src % 2 == 0);
  const bool mfma = j.ldtype == kBF16 && lb == 15 && aligned;
  return ClassKey{mfma, j.ldtype, mfma ? kBF16 : j.wdtype, lb, mfma ? j.layers : 0};
}

// Partial rows of the backward: bfloat16 for the matrix-core chain (as in its
// per-module launch), float32 otherwise; 128-byte aligned, so n is rounded up
// to 64 bfloat16 or 32 float32 values.
bool part_bf16(const WeightJob& j) { return class_of(j, false).mfma; }
int64_t row_stride(const WeightJob& j) { return part_bf16(j) ? (j.n + 63) / 64 * 64 : (j.n + 31) / 32 * 32; }
size_t row_bytes(const WeightJob& j) { return (size_t)row_stride(j) * (part_bf16(j) ? 2 : 4); }

size_t partial_bytes(const WeightJob& j);

int64_t blocks_of(const WeightJob& j) {
  const int64_t B = (int64_t)1 << log2_ceil(j.n);
  return (j.size + B - 1) / B;
}

// Workgroups of one job in its class's kernel.
int64_t workgroups_of(const ClassKey& k, const WeightJob& j) {
  if (k.mfma) return blocks_of(j);
  const int g = group_slots_per_wg(k.log_block);
  return (blocks_of(j) + g - 1) / g;
}

size_t partial_bytes(const WeightJob& j) { return align_up((size_t)blocks_of(j) * row_bytes(j)); }

GroupJob device_job(const WeightJob& j, bool fwd, void* part) {
  GroupJob d{};
  d.src = fwd ? j.latent : j.grad_weight;
  d.dst = fwd ? j.weight : j.grad_latent;
  d.part = part;
  d.size = j.size;
  d.n = (int32_t)j.n;
  d.stride = (int32_t)row_stride(j);
  d.part_bf16 = !fwd && part_bf16(j);
  d.nblocks = (int32_t)blocks_of(j);
  d.seed32 = j.seed32;
  d.layers = j.layers;
  d.wdtype = j.wdtype;
  d.accumulate = j.accumulate;
  d.scale = j.scale;
  return d;
}

// Runs `launch` over the jobs in `idx` in tables of up to kGroupMaxJobs jobs;
// units(j) is the job's share of the grid.
template <class Units, class Launch>
hipError_t run_tables(const std::vector<int>& idx, const std::vector<GroupJob>& djobs, Units units,
                      Launch launch) {
  GroupTable t{};
  auto flush = [&]() -> hipError_t {
    if (t.count == 0) return hipSuccess;
    const hipError_t e = launch(t);
    t = GroupTable{};
    return e;
  };
  for (int i : idx) {
    const int64_t u = units(i);
    if (t.count == kGroupMaxJobs || (int64_t)t.prefix[t.count] + u > kGroupMaxGrid) {
      const hipError_t e = flush();
      if (e != hipSuccess) return e;
    }
    t.job[t.count] = djobs[i];
    t.prefix[t.count + 1] = t.prefix[t.count] + (int32_t)u;
    ++t.count;
  }
  return flush();
}

}  // namespace

bool grouped_job_supported(const WeightJob& j, bool fwd, const char** why) {
  if (log2_ceil(j.n) > kWholeBlockMaxLog) {
    *why = "grouped weight calls take blocks up to 2^15 (latent size <= 32768)";
    return false;
  }
  if (class_of(j, fwd).mfma && j.wdtype != kBF16) {
    *why = "bfloat16 latents of block 2^15 need a bfloat16 weight in grouped weight calls";
    return false;
  }
  if (blocks_of(j) > kGroupMaxGrid || workgroups_of(class_of(j, fwd), j) > kGroupMaxGrid) {
    *why = "weight too large for one grouped launch";
    return false;
  }
  return true;
}

size_t grouped_workspace_bytes(const WeightJob* jobs, int64_t count) {
  size_t total = 0;
  for (int64_t i = 0; i < count; ++i) total += partial_bytes(jobs[i]);
  return total;
}

hipError_t launch_grouped(const WeightJob* jobs, int64_t count, void* work, hipStream_t s, bool fwd) {
  std::vector<GroupJob> djobs((size_t)count);
  std::vector<ClassKey> keys((size_t)count);
  size_t off = 0;
  for (int64_t i = 0; i < count; ++i) {
    void* part = nullptr;
    if (!fwd) {
      part = static_cast<char*>(work) + off;
      off += partial_bytes(jobs[i]);
    }
    djobs[i] = device_job(jobs[i], fwd, part);
    keys[i] = class_of(jobs[i], fwd);
  }
  // classes in order of first appearance
  std::vector<bool> done((size_t)count, false);
  for (int64_t i = 0; i < count; ++i) {
    if (done[i]) continue;
    const ClassKey k = keys[i];
    std::vector<int> idx;
    for (int64_t m = i; m < count; ++m)
      if (!done[m] && keys[m] == k) {
        idx.push_back((int)m);
        done[m] = true;
      }
    const hipError_t e = run_tables(
        idx, djobs, [&](int m) { return workgroups_of(k, jobs[m]); },
        [&](const GroupTable& t) {
          return k.mfma ? launch_mfma15_grouped(t, k.layers, s, fwd)
                        : launch_block_grouped(t, k.dtype, k.wdtype, k.log_block, s, fwd);
        });
    if (e != hipSuccess) return e;
  }
  if (fwd) return hipSuccess;
  // fixed-order block sums with the scale / accumulate epilogue, per latent
  // dtype and partial-row type
  for (int dtype : {kF32, kF16, kBF16})
    for (bool bf16_rows : {false, true}) {
      std::vector<int> idx;
      for (int64_t m = 0; m < count; ++m)
        if (jobs[m].ldtype == dtype && part_bf16(jobs[m]) == bf16_rows) idx.push_back((int)m);
      const hipError_t e = run_tables(
          idx, djobs, [&](int m) { return (jobs[m].n + kGroupReduceCols - 1) / kGroupReduceCols; },
          [&](const GroupTable& t) { return launch_reduce_grouped(t, dtype, bf16_rows, s); });
      if (e != hipSuccess) return e;
    }
  return hipSuccess;
}

}  // namespace lwl
