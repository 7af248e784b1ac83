// Stage handoff probe: what one dependent stage costs as a kernel boundary
// (S launches in a HIP graph) and as a grid-wide handoff inside one launch.
// A measurement program for bench.py (`--only handoff`), not part of the
// library.  It bounds any design that chains the latent and expand stages of
// consecutive projections inside one persistent launch.
//
// Work per stage, the same in both forms: every block writes kD floats of its
// output for stage s, each the sum of kRead other blocks' stage s - 1 values.
//
//   boundary form: stage_kernel launched S times in one graph.
//   handoff form:  handoff_kernel runs the S stages in one launch.  Between
//     stages each block stores its output with agent-scope stores (written
//     through to the point every XCD reads), waits for them (vmcnt 0), adds 1
//     to one of nc counters (non-returning, agent scope, each counter on its
//     own 128-byte line), and its first wave polls the stage's nc counters
//     (one agent-scope load per lane) until they sum to the block count; the
//     next stage reads with agent-scope loads.  No fences.
//
// Safety: the grid never exceeds the resident capacity (occupancy query x
// CUs), and every poll loop is bounded: past spin_max polls a block sets the
// abort flag, and every block leaves at its next poll.  The program also runs
// the handoff form with spin_max = 1 and checks that it ends with the flag
// set.  Output: one JSON line.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x)                                                                                   \
  do {                                                                                             \
    hipError_t e_ = (x);                                                                           \
    if (e_ != hipSuccess) {                                                                        \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_));            \
      exit(1);                                                                                     \
    }                                                                                              \
  } while (0)

namespace {

constexpr int kD = 64;        // floats per block output
constexpr int kRead = 4;      // other blocks' outputs summed per stage
constexpr int kLine = 32;     // uint32 per counter slot: 128 bytes
constexpr int kMaxCounters = 32;  // lane kMaxCounters of the polling wave reads the abort flag
constexpr int kSpinMax = 1 << 20;

__device__ __forceinline__ float stage_value(const float* __restrict__ prev, int nb, int b, int s, int lane,
                                             bool agent) {
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < kRead; ++i) {
    const int src = (b * 7 + i * 13 + s) % nb;
    const float* q = prev + size_t(src) * kD + lane;
    acc += agent ? __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *q;
  }
  return acc * 0.5f + float(b);
}

__global__ __launch_bounds__(256) void stage_kernel(float* __restrict__ buf, int nb, int s) {
  const int b = int(blockIdx.x), lane = int(threadIdx.x);
  if (lane >= kD) return;
  const float* prev = buf + size_t(s & 1) * nb * kD;
  float* cur = buf + size_t((s + 1) & 1) * nb * kD;
  cur[size_t(b) * kD + lane] = stage_value(prev, nb, b, s, lane, false);
}

// cnt: [S][nc][kLine] uint32, zero on entry; abort_flag: one uint32, zero on entry
__global__ __launch_bounds__(256) void handoff_kernel(float* __restrict__ buf, int nb, int S, int nc,
                                                      uint32_t* __restrict__ cnt, uint32_t* __restrict__ abort_flag,
                                                      int spin_max) {
  const int b = int(blockIdx.x), tid = int(threadIdx.x);
  __shared__ int s_ok;
  for (int s = 0; s < S; ++s) {
    const float* prev = buf + size_t(s & 1) * nb * kD;
    float* cur = buf + size_t((s + 1) & 1) * nb * kD;
    if (tid < kD) {
      const float v = stage_value(prev, nb, b, s, tid, true);
      __hip_atomic_store(cur + size_t(b) * kD + tid, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
    __syncthreads();
    if (tid == 0)
      __hip_atomic_fetch_add(cnt + (size_t(s) * nc + (b % nc)) * kLine, 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    if (tid < 64) {
      int ok = 0;
      for (int it = 0; it < spin_max; ++it) {
        uint32_t v = 0;
        if (tid < nc)
          v = __hip_atomic_load(cnt + (size_t(s) * nc + tid) * kLine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else if (tid == nc)
          v = __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t ab = __shfl(v, nc);
        uint32_t sum = tid < nc ? v : 0u;
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        if (ab) break;
        if (sum >= uint32_t(nb)) {
          ok = 1;
          break;
        }
        if (it + 1 == spin_max && tid == 0)
          __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (tid == 0) s_ok = ok;
    }
    __syncthreads();
    if (!s_ok) return;  // the whole block
  }
}

float median(std::vector<float> v) {
  std::sort(v.begin(), v.end());
  return v[v.size() / 2];
}

}  // namespace

int main(int argc, char** argv) {
  const int S = argc > 1 ? std::max(1, atoi(argv[1])) : 64;
  int dev = 0, ncu = 0, occ = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
  CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, handoff_kernel, 256, 0));
  hipStream_t st;
  CHECK(hipStreamCreate(&st));
  const int maxnb = ncu * std::min(occ, 2);
  float* buf;
  uint32_t *cnt, *abort_flag;
  CHECK(hipMalloc(&buf, size_t(2) * maxnb * kD * sizeof(float)));
  CHECK(hipMemset(buf, 0, size_t(2) * maxnb * kD * sizeof(float)));
  CHECK(hipMalloc(&cnt, size_t(S) * kMaxCounters * kLine * sizeof(uint32_t)));
  CHECK(hipMalloc(&abort_flag, sizeof(uint32_t)));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  printf("{\"stages\": %d, \"cus\": %d, \"resident_blocks_per_cu\": %d, \"runs\": [", S, ncu, occ);
  bool first = true;
  for (int nb : {ncu, maxnb}) {
    if (nb > ncu * occ) continue;
    hipGraph_t g;
    hipGraphExec_t ge;
    CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    for (int s = 0; s < S; ++s) hipLaunchKernelGGL(stage_kernel, dim3(nb), dim3(256), 0, st, buf, nb, s);
    CHECK(hipStreamEndCapture(st, &g));
    CHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    for (int w = 0; w < 3; ++w) CHECK(hipGraphLaunch(ge, st));
    CHECK(hipStreamSynchronize(st));
    std::vector<float> tb;
    for (int r = 0; r < 7; ++r) {
      CHECK(hipEventRecord(e0, st));
      CHECK(hipGraphLaunch(ge, st));
      CHECK(hipEventRecord(e1, st));
      CHECK(hipEventSynchronize(e1));
      float ms;
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      tb.push_back(ms * 1000.f / S);
    }
    CHECK(hipGraphExecDestroy(ge));
    CHECK(hipGraphDestroy(g));
    printf("%s{\"blocks\": %d, \"boundary_us_per_stage\": %.3f, \"handoff_us_per_stage\": {", first ? "" : ", ", nb,
           median(tb));
    first = false;
    for (int nc : {8, 16, 32}) {
      std::vector<float> th;
      int aborted = 0;
      for (int r = 0; r < 8; ++r) {
        CHECK(hipMemsetAsync(cnt, 0, size_t(S) * nc * kLine * sizeof(uint32_t), st));
        CHECK(hipMemsetAsync(abort_flag, 0, sizeof(uint32_t), st));
        CHECK(hipEventRecord(e0, st));
        hipLaunchKernelGGL(handoff_kernel, dim3(nb), dim3(256), 0, st, buf, nb, S, nc, cnt, abort_flag, kSpinMax);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(e1, st));
        CHECK(hipEventSynchronize(e1));
        uint32_t ab = 0;
        CHECK(hipMemcpy(&ab, abort_flag, 4, hipMemcpyDeviceToHost));
        aborted += ab != 0;
        float ms;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        if (r > 0) th.push_back(ms * 1000.f / S);
      }
      printf("%s\"%d_counters\": %s", nc == 8 ? "" : ", ", nc, aborted ? "null" : "");
      if (!aborted) printf("%.3f", median(th));
    }
    // the give-up path: one poll per wait must still end every block
    CHECK(hipMemsetAsync(cnt, 0, size_t(S) * 8 * kLine * sizeof(uint32_t), st));
    CHECK(hipMemsetAsync(abort_flag, 0, sizeof(uint32_t), st));
    hipLaunchKernelGGL(handoff_kernel, dim3(nb), dim3(256), 0, st, buf, nb, S, 8, cnt, abort_flag, 1);
    CHECK(hipStreamSynchronize(st));
    uint32_t ab = 0;
    CHECK(hipMemcpy(&ab, abort_flag, 4, hipMemcpyDeviceToHost));
    printf("}, \"spin_limit_1_ended_with_abort\": %s}", ab ? "true" : "false");
  }
  printf("]}\n");
  return 0;
}
