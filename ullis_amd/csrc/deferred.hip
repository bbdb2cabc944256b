// Batched end-of-step parameter updates: one launch per kind of update for
// every tensor of a train step (job tables in ops.hpp). Each block finds its
// job by a scan of the job table, then runs the same per-tensor body as the
// immediate launchers (update.hpp), so results are identical to updating each
// tensor right after its gradient is complete.
#include "common.hpp"
#include "ops.hpp"
#include "update.hpp"

namespace ullis {

namespace {

template <class J>
__device__ __forceinline__ int find_job(const J* jobs, int njobs, int blk) {
  int j = 0;
  while (j + 1 < njobs && jobs[j + 1].block0 <= blk) ++j;
  return j;
}

__global__ __launch_bounds__(1024) void vec_jobs_kernel(const VecJob* jobs, int njobs, float lr,
                                                        const uint32_t* abort) {
  __shared__ float red[64][64];
  if (abort && *abort) return;
  const int j = find_job(jobs, njobs, blockIdx.x);
  const VecJob& jb = jobs[j];
  vec_reduce_block(jb.part, jb.nblk, jb.ncols, jb.split, jb.a, jb.a.lr * lr, jb.b, jb.b.lr * lr,
                   (long)blockIdx.x - jb.block0, red);
}

__global__ __launch_bounds__(256) void finish_jobs_kernel(const FinishJob* jobs, int njobs,
                                                          float lr, const uint32_t* abort) {
  const int j = find_job(jobs, njobs, blockIdx.x);
  const PackedFinish f = jobs[j].f;
  const long o = ((long)blockIdx.x - jobs[j].block0) * 4 + (threadIdx.x >> 6);
  if (o >= f.out) return;
  if (abort && *abort) {  // refused step: nothing changes
    if ((threadIdx.x & 63) == 0) {
      if (f.row_flips) f.row_flips[o] = 0;
      if (f.row_step) f.row_step[o] = 0.0f;
    }
    return;
  }
  packed_finish_row_wave(f, o, lr);
}

__global__ __launch_bounds__(256) void f16_jobs_kernel(const F16Job* jobs, int njobs, float lr,
                                                       const uint32_t* abort) {
  if (abort && *abort) return;
  const int j = find_job(jobs, njobs, blockIdx.x);
  const F16Job& jb = jobs[j];
  const long i = (((long)blockIdx.x - jb.block0) * blockDim.x + threadIdx.x) * 4;
  if (i < jb.n) fp16_finish_four(jb.part, jb.splits, jb.n, i, jb.amax, lr, jb.w, jb.w_res, nullptr);
}

__global__ __launch_bounds__(256) void trans_jobs_kernel(const TransJob* jobs, int njobs,
                                                         const uint32_t* abort) {
  if (abort && *abort) return;
  const int j = find_job(jobs, njobs, blockIdx.x);
  const TransJob& jb = jobs[j];
  const long blk = (((long)blockIdx.x - jb.block0) * blockDim.x + threadIdx.x) >> 5;
  transpose_bits_block(jb.bits, jb.out, jb.in, jb.bits_t, blk,
                       blk < (jb.out / 32) * (jb.in / 32));
}

}  // namespace

hipError_t run_vec_jobs(hipStream_t s, const VecJob* jobs, int njobs, int nblocks, float lr,
                        const uint32_t* abort) {
  if (njobs <= 0 || nblocks <= 0) return hipSuccess;
  launch(vec_jobs_kernel, dim3((unsigned)nblocks), dim3(1024), 0, s, jobs, njobs, lr, abort);
  return hipGetLastError();
}

hipError_t run_finish_jobs(hipStream_t s, const FinishJob* jobs, int njobs, int nblocks,
                           float lr, const uint32_t* abort) {
  if (njobs <= 0 || nblocks <= 0) return hipSuccess;
  launch(finish_jobs_kernel, dim3((unsigned)nblocks), dim3(256), 0, s, jobs, njobs, lr, abort);
  return hipGetLastError();
}

hipError_t run_f16_jobs(hipStream_t s, const F16Job* jobs, int njobs, int nblocks, float lr,
                        const uint32_t* abort) {
  if (njobs <= 0 || nblocks <= 0) return hipSuccess;
  launch(f16_jobs_kernel, dim3((unsigned)nblocks), dim3(256), 0, s, jobs, njobs, lr, abort);
  return hipGetLastError();
}

hipError_t run_trans_jobs(hipStream_t s, const TransJob* jobs, int njobs, int nblocks,
                          const uint32_t* abort) {
  if (njobs <= 0 || nblocks <= 0) return hipSuccess;
  launch(trans_jobs_kernel, dim3((unsigned)nblocks), dim3(256), 0, s, jobs, njobs, abort);
  return hipGetLastError();
}

}  // namespace ullis
