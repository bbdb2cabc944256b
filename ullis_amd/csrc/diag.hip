// The step diagnostics the reference's train_step_on returns with its loss
// (CausalLoss, src/model.rs:58-80, filled at src/model.rs:2997-3024), computed
// on the device from the step's outputs and the updated parameters, so a
// caller that logs them every step (src/main.rs) downloads one small struct
// instead of the head's sign bits, latents and row losses.
//
//  - loss percentiles (loss_percentiles, src/model.rs:3341-3363): the finite
//    row losses of valid rows, ranked under f32::total_cmp; the p-th value is
//    the one at rank min(round(p (n - 1)), n - 1). Each row's rank is counted
//    against every other row (rank = #smaller + #equal earlier rows), so the
//    selection is exact and needs no sort;
//  - unigram CE (unigram_cross_entropy, src/model.rs:3365-3390): target counts
//    by integer atomics, then -sum count ln(count / n) / n;
//  - flip counts (bit_flip_count, src/model.rs:150-156): the per-row counts the
//    packed finish kernels wrote during the step, summed per class;
//  - rms / mean-abs statistics (src/model.rs:3293-3339): fixed-order two-stage
//    sums (the reference sums sequentially; the values agree to rounding).
#include "common.hpp"
#include "context.hpp"
#include "ops.hpp"

namespace ullis {

namespace {

struct DiagTaskTable {
  DiagTask t[kDiagMaxTasks];
};

__global__ void diag_tasks_store_kernel(DiagTaskTable table, int n, DiagTask* dst) {
  if ((int)threadIdx.x < n) dst[threadIdx.x] = table.t[threadIdx.x];
}

constexpr int kDiagBlocks = 64;  // blocks per reduction task
constexpr int kDiagThreads = 256;

__device__ __forceinline__ float task_term(const DiagTask& t, long i) {
  switch (t.kind) {
    case DiagTask::kSqF32: {
      const float v = static_cast<const float*>(t.p)[i];
      return v * v;
    }
    case DiagTask::kAbsF32:
      return __builtin_fabsf(static_cast<const float*>(t.p)[i]);
    case DiagTask::kSqF16: {
      const float v = f16_bits_to_f32(static_cast<const uint16_t*>(t.p)[i]);
      return v * v;
    }
    case DiagTask::kAbsF16:
      return __builtin_fabsf(f16_bits_to_f32(static_cast<const uint16_t*>(t.p)[i]));
    case DiagTask::kSumF32:
      return static_cast<const float*>(t.p)[i];
    default:
      return 0.0f;
  }
}

// Block b of task blockIdx.y sums elements b * 256 + t, stride 64 * 256, then
// a fixed tree over the block; float tasks into fpart, count tasks into upart.
__global__ __launch_bounds__(kDiagThreads) void diag_sums_kernel(const DiagTask* tasks,
                                                                 float* fpart,
                                                                 unsigned long long* upart) {
  __shared__ float fs[kDiagThreads];
  __shared__ unsigned long long us[kDiagThreads];
  const DiagTask t = tasks[blockIdx.y];
  float f = 0.0f;
  unsigned long long u = 0;
  for (long i = (long)blockIdx.x * kDiagThreads + threadIdx.x; i < t.n;
       i += (long)kDiagBlocks * kDiagThreads) {
    if (t.kind == DiagTask::kSumU32)
      u += static_cast<const uint32_t*>(t.p)[i];
    else
      f += task_term(t, i);
  }
  fs[threadIdx.x] = f;
  us[threadIdx.x] = u;
  __syncthreads();
  for (int st = kDiagThreads / 2; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st) {
      fs[threadIdx.x] += fs[threadIdx.x + st];
      us[threadIdx.x] += us[threadIdx.x + st];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    fpart[blockIdx.y * kDiagBlocks + blockIdx.x] = fs[0];
    upart[blockIdx.y * kDiagBlocks + blockIdx.x] = us[0];
  }
}

// Valid rows (causal_ce_row_valid with horizon 1, targets < vocab) whose loss
// is finite: their targets are counted into counts[vocab] and their number
// into *n_rank.
__global__ __launch_bounds__(256) void diag_rows_kernel(const float* row_loss,
                                                        const uint32_t* targets, long rows,
                                                        long time, long vocab, uint32_t ignore_id,
                                                        uint32_t* counts, uint32_t* n_valid,
                                                        uint32_t* n_rank) {
  const long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
  bool valid = false, ranked = false;
  if (r < rows && r % time + 1 < time && r + 1 < rows) {
    const uint32_t id = targets[r + 1];
    valid = id != ignore_id && (long)id < vocab;
    if (valid) {
      atomicAdd(counts + id, 1u);
      ranked = __builtin_isfinite(row_loss[r]);
    }
  }
  const unsigned long long mv = __ballot(valid), mr = __ballot(ranked);
  if ((threadIdx.x & 63) == 0) {
    if (mv) atomicAdd(n_valid, (uint32_t)__popcll(mv));
    if (mr) atomicAdd(n_rank, (uint32_t)__popcll(mr));
  }
}

// f32::total_cmp order as an unsigned key.
__device__ __forceinline__ uint32_t total_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Key of row j, or 0 (never compared) when row j is not ranked.
__device__ __forceinline__ uint32_t rank_key(const float* row_loss, const uint32_t* targets,
                                             long j, long rows, long time, long vocab,
                                             uint32_t ignore_id, bool& ranked) {
  ranked = false;
  if (j < rows && j % time + 1 < time && j + 1 < rows) {
    const uint32_t id = targets[j + 1];
    if (id != ignore_id && (long)id < vocab && __builtin_isfinite(row_loss[j])) {
      ranked = true;
      return total_key(row_loss[j]);
    }
  }
  return 0u;
}

// Every ranked row i counts the ranked rows before it in (key, row) order; the
// rows whose rank is a percentile's index write their loss.
__global__ __launch_bounds__(256) void diag_rank_kernel(const float* row_loss,
                                                        const uint32_t* targets, long rows,
                                                        long time, long vocab, uint32_t ignore_id,
                                                        const uint32_t* n_rank, float* pct) {
  constexpr int kTile = 2048;
  __shared__ uint32_t keys[kTile];
  __shared__ unsigned char ok[kTile];
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  bool mine = false;
  const uint32_t ki = rank_key(row_loss, targets, i, rows, time, vocab, ignore_id, mine);
  const long n = (long)*n_rank;
  long rank = 0;
  for (long j0 = 0; j0 < rows; j0 += kTile) {
    __syncthreads();
    for (int t = threadIdx.x; t < kTile; t += blockDim.x) {
      bool r = false;
      keys[t] = rank_key(row_loss, targets, j0 + t, rows, time, vocab, ignore_id, r);
      ok[t] = r ? 1 : 0;
    }
    __syncthreads();
    if (mine) {
      const long m = rows - j0 < kTile ? rows - j0 : kTile;
      for (int t = 0; t < m; ++t) {
        const uint32_t kj = keys[t];
        rank += (ok[t] && (kj < ki || (kj == ki && j0 + t < i))) ? 1 : 0;
      }
    }
  }
  if (!mine || n == 0) return;
  const float ps[3] = {0.10f, 0.50f, 0.90f};
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    long at = (long)__builtin_roundf(ps[q] * (float)(n - 1));
    if (at > n - 1) at = n - 1;
    if (rank == at) pct[q] = row_loss[i];
  }
}

// Terms of the unigram CE: count * ln(count / n) over targets that occur.
__global__ __launch_bounds__(kDiagThreads) void diag_unigram_kernel(const uint32_t* counts,
                                                                    long vocab,
                                                                    const uint32_t* n_valid,
                                                                    float* fpart,
                                                                    unsigned long long* upart) {
  __shared__ float fs[kDiagThreads];
  __shared__ unsigned long long us[kDiagThreads];
  const float n = (float)*n_valid;
  float f = 0.0f;
  unsigned long long u = 0;
  for (long v = (long)blockIdx.x * kDiagThreads + threadIdx.x; v < vocab;
       v += (long)kDiagBlocks * kDiagThreads) {
    const uint32_t c = counts[v];
    if (c) {
      const float p = (float)c / n;
      f += (float)c * __builtin_logf(p);
      u += 1;
    }
  }
  fs[threadIdx.x] = f;
  us[threadIdx.x] = u;
  __syncthreads();
  for (int st = kDiagThreads / 2; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st) {
      fs[threadIdx.x] += fs[threadIdx.x + st];
      us[threadIdx.x] += us[threadIdx.x + st];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    fpart[blockIdx.x] = fs[0];
    upart[blockIdx.x] = us[0];
  }
}

__device__ __forceinline__ float sum_parts(const float* p) {
  float s = 0.0f;
  for (int b = 0; b < kDiagBlocks; ++b) s += p[b];
  return s;
}
__device__ __forceinline__ unsigned long long sum_parts(const unsigned long long* p) {
  unsigned long long s = 0;
  for (int b = 0; b < kDiagBlocks; ++b) s += p[b];
  return s;
}

__global__ void diag_finish_kernel(const DiagTask* tasks, int ntasks, const float* fpart,
                                   const unsigned long long* upart, const float* uni_f,
                                   const unsigned long long* uni_u, const uint32_t* n_valid,
                                   const float* pct, const float* stats, DiagOut out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  float* o = reinterpret_cast<float*>(out.dst);
  uint32_t* ou = reinterpret_cast<uint32_t*>(out.dst);
  const float n = (float)*n_valid;
  o[kDiagNextToken] = stats[0];
  ou[kDiagNextTokenCount] = *n_valid;
  o[kDiagP10] = pct[0];
  o[kDiagP50] = pct[1];
  o[kDiagP90] = pct[2];
  o[kDiagUnigramCe] = *n_valid ? -sum_parts(uni_f) / n : 0.0f;
  ou[kDiagUniqueTargets] = *n_valid ? (uint32_t)sum_parts(uni_u) : 0u;
  unsigned long long flips = 0;
  for (int k = 0; k < ntasks; ++k) {
    const DiagTask& t = tasks[k];
    if (t.field < 0) continue;
    if (t.kind == DiagTask::kSumU32) {
      const unsigned long long c = sum_parts(upart + k * kDiagBlocks);
      ou[t.field] = (uint32_t)c;
      flips += c;
      continue;
    }
    const float s = sum_parts(fpart + k * kDiagBlocks);
    const float m = t.n > 0 ? s / (float)t.denom : 0.0f;
    o[t.field] = t.rms ? __builtin_sqrtf(m) : m;
  }
  ou[kDiagFlipsTotal] = (uint32_t)flips;
}

}  // namespace

size_t diag_workspace_bytes(long vocab) {
  return Carver::bytes_for(sizeof(DiagTask) * kDiagMaxTasks) +
         Carver::bytes_for(sizeof(float) * kDiagMaxTasks * kDiagBlocks) +
         Carver::bytes_for(sizeof(unsigned long long) * kDiagMaxTasks * kDiagBlocks) +
         Carver::bytes_for(sizeof(float) * kDiagBlocks) +
         Carver::bytes_for(sizeof(unsigned long long) * kDiagBlocks) +
         Carver::bytes_for(sizeof(uint32_t) * 4) + Carver::bytes_for(sizeof(float) * 4) +
         Carver::bytes_for(sizeof(uint32_t) * vocab);
}

hipError_t causal_loss_diag(hipStream_t s, const DiagArgs& a, const DiagTask* tasks_host,
                            int ntasks, void* workspace) {
  if (ntasks > kDiagMaxTasks || a.rows <= 0 || a.vocab <= 0 || a.time < 2)
    return hipErrorInvalidValue;
  Carver cv(workspace);
  DiagTask* tasks = cv.take<DiagTask>(kDiagMaxTasks);
  float* fpart = cv.take<float>(kDiagMaxTasks * kDiagBlocks);
  unsigned long long* upart = cv.take<unsigned long long>(kDiagMaxTasks * kDiagBlocks);
  float* uni_f = cv.take<float>(kDiagBlocks);
  unsigned long long* uni_u = cv.take<unsigned long long>(kDiagBlocks);
  uint32_t* cnt = cv.take<uint32_t>(4);  // n_valid, n_rank
  float* pct = cv.take<float>(4);
  uint32_t* counts = cv.take<uint32_t>(a.vocab);
  hipError_t e;
  // the task table travels as a kernel-argument copy: no host-to-device copy
  // of pageable memory inside a stream the caller may capture
  DiagTaskTable table{};
  for (int k = 0; k < ntasks; ++k) table.t[k] = tasks_host[k];
  launch(diag_tasks_store_kernel, dim3(1), dim3(kDiagMaxTasks), 0, s, table, ntasks, tasks);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if ((e = fill_f32(s, reinterpret_cast<float*>(cnt), 2, 0.0f)) != hipSuccess) return e;
  if ((e = fill_f32(s, pct, 3, 0.0f)) != hipSuccess) return e;
  if ((e = fill_f32(s, reinterpret_cast<float*>(counts), a.vocab, 0.0f)) != hipSuccess) return e;
  launch(diag_rows_kernel, dim3((unsigned)cdiv(a.rows, 256)), dim3(256), 0, s, a.row_loss,
         a.targets, a.rows, a.time, a.vocab, a.ignore_id, counts, cnt, cnt + 1);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (ntasks > 0) {
    launch(diag_sums_kernel, dim3(kDiagBlocks, (unsigned)ntasks), dim3(kDiagThreads), 0, s,
           (const DiagTask*)tasks, fpart, upart);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  launch(diag_rank_kernel, dim3((unsigned)cdiv(a.rows, 256)), dim3(256), 0, s, a.row_loss,
         a.targets, a.rows, a.time, a.vocab, a.ignore_id, (const uint32_t*)(cnt + 1), pct);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  launch(diag_unigram_kernel, dim3(kDiagBlocks), dim3(kDiagThreads), 0, s,
         (const uint32_t*)counts, a.vocab, (const uint32_t*)cnt, uni_f, uni_u);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  launch(diag_finish_kernel, dim3(1), dim3(64), 0, s, (const DiagTask*)tasks, ntasks,
         (const float*)fpart, (const unsigned long long*)upart, (const float*)uni_f,
         (const unsigned long long*)uni_u, (const uint32_t*)cnt, (const float*)pct, a.stats,
         DiagOut{a.out});
  return hipGetLastError();
}

}  // namespace ullis
