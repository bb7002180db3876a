// Library-wide C entry points: version, error reporting, device queries and the
// indexer schedule.
#include <cstdarg>
#include <cstdio>

#include "dsa_common.h"
#include "../../include/dsa_amd.h"

namespace dsa {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(kLaunchFailed, "%s: launch failed: %s", what, hipGetErrorString(e));
  return kOk;
}

// Exclusive prefix sum of per-sequence page counts; one thread block scans
// serially in chunks of 1024 (the batch is small: one entry per sequence).
__global__ void __launch_bounds__(1024) indexer_schedule_kernel(const int32_t* __restrict__ ctx, int batch,
                                                                int next_n, int page_size,
                                                                int32_t* __restrict__ out) {
  __shared__ int32_t s_part[1024];
  __shared__ int32_t s_carry;
  if (threadIdx.x == 0) s_carry = 0;
  __syncthreads();
  for (int base = 0; base < batch; base += 1024) {
    int b = base + (int)threadIdx.x;
    int pages = 0;
    if (b < batch) {
      int L = 0;
      for (int j = 0; j < next_n; ++j) L = max(L, ctx[(int64_t)b * next_n + j]);
      pages = (max(L, 0) + page_size - 1) / page_size;
    }
    s_part[threadIdx.x] = pages;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      int v = threadIdx.x >= (unsigned)off ? s_part[threadIdx.x - off] : 0;
      __syncthreads();
      s_part[threadIdx.x] += v;
      __syncthreads();
    }
    if (b < batch) out[b] = s_carry + s_part[threadIdx.x] - pages;
    __syncthreads();
    if (threadIdx.x == 1023) s_carry += s_part[1023];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[batch] = s_carry;
}

}  // namespace dsa

extern "C" {

int dsa_version(void) { return 100; }

const char* dsa_last_error(void) { return dsa::g_last_error; }

int dsa_num_cus(int device) {
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return -1;
  return n;
}

int dsa_indexer_schedule(const int32_t* context_lens, int batch, int next_n, int page_size,
                         int32_t* schedule_out, void* stream) {
  if (batch < 0 || next_n < 1 || page_size <= 0 || !schedule_out || (batch > 0 && !context_lens))
    return dsa::set_error(dsa::kInvalidArgument, "dsa_indexer_schedule: bad arguments");
  hipLaunchKernelGGL(dsa::indexer_schedule_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream,
                     context_lens, batch, next_n, page_size, schedule_out);
  return dsa::check_launch("dsa_indexer_schedule");
}

}  // extern "C"
