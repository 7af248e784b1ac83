// Issue-rate probe for the GEMM path's mainloop on gfx950: how much the VALU
// work and the LDS reads that feed 32x32x16 bf16 MFMAs cost the MFMA pipe.
// A standalone program (bench.py --only issue runs it as a child process);
// it prints one JSON line per case.
//
//   valu  V: each wave runs rounds of 8 independent MFMAs (8 accumulator
//            sets) with V independent VALU instructions after each MFMA;
//            "dep" variants make those VALU rewrite the next MFMA's B
//            operand, as the in-register sign expansion does.
//   lds   U: each 1 KB A fragment read from LDS (ds_read_b128) feeds U MFMAs;
//            U = 0 reads only (LDS read bandwidth).
//   ring:    the GEMM mainloop's skeleton without the sign expansion
//            (ring_kernel below), with and without the A-tile loads.
//
// Grids: 256 threads per block, 256 blocks (one wave per SIMD on 256 CUs),
// 512 (two) and 768 (three; not for ring, whose 64 KB of LDS fit two blocks
// per CU).
// The valu and lds cases use only registers and LDS; ring reads a 4 MiB
// buffer, every address inside it.  Each thread stores one float at the end,
// into a buffer of exactly grid x 256 floats.
#include <hip/hip_runtime.h>

#include <cstdio>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMaxBlocks = 768;

template <int V, bool DEP>
__global__ __launch_bounds__(kThreads, 2) void valu_kernel(float* out, int iters) {
  f32x16 acc[8];
  for (int m = 0; m < 8; ++m) acc[m] = f32x16{};
  const unsigned tid = threadIdx.x;
  unsigned x0 = tid, x1 = tid * 3u, x2 = tid * 5u, x3 = tid * 7u;
  unsigned b0 = 0x3F803F80u ^ (x0 << 15), b1 = 0x3F803F80u, b2 = 0x3F803F80u, b3 = 0x3F803F80u ^ (x1 << 31);
  const u32x4 a = {0x3F803F80u, 0x3F803F80u ^ (x2 << 15), 0x3F803F80u, 0x3F803F80u};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, (u32x4{b0, b1, b2, b3})), acc[m],
                                                       0, 0, 0);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if constexpr (DEP) {
          unsigned& d = (v & 3) == 0 ? b0 : (v & 3) == 1 ? b1 : (v & 3) == 2 ? b2 : b3;
          asm volatile("v_xor_b32 %0, %0, %1" : "+v"(d) : "v"(x0));
        } else {
          unsigned& d = (v & 3) == 0 ? x0 : (v & 3) == 1 ? x1 : (v & 3) == 2 ? x2 : x3;
          asm volatile("v_add_u32 %0, %0, %1" : "+v"(d) : "v"(x3));
        }
      }
    }
  }
  float s = 0.f;
  for (int m = 0; m < 8; ++m)
    for (int e = 0; e < 16; ++e) s += acc[m][e];
  out[blockIdx.x * kThreads + tid] = s + float(x0 ^ x1 ^ x2 ^ x3) + float(b0 ^ b3);
}

template <int U>
__global__ __launch_bounds__(kThreads, 2) void lds_kernel(float* out, int iters) {
  __shared__ u32x4 lds[1024];  // 16 KB: 16 fragments of 1 KB
  const int tid = int(threadIdx.x);
  for (int i = tid; i < 1024; i += kThreads) lds[i] = u32x4{0x3F803F80u, 0x3F803F80u ^ unsigned(i), 0x3F803F80u, 0u};
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6;
  f32x16 acc[8];
  for (int m = 0; m < 8; ++m) acc[m] = f32x16{};
  u32x4 x = {0u, 0u, 0u, 0u};
  const u32x4 b = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u ^ unsigned(lane << 15), 0x3F803F80u};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int slot = ((it * 8 + m) * 5 + wave * 3) & 15;  // in [0, 16)
      const u32x4 a = lds[slot * 64 + lane];
      if constexpr (U == 0) {
        x ^= a;
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u)
          acc[(m * U + u) & 7] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc[(m * U + u) & 7], 0, 0, 0);
      }
    }
  }
  float s = float(x[0] ^ x[1] ^ x[2] ^ x[3]);
  for (int m = 0; m < 8; ++m)
    for (int e = 0; e < 16; ++e) s += acc[m][e];
  out[blockIdx.x * kThreads + tid] = s;
}

// The GEMM mainloop's skeleton without the sign expansion: 4 waves, a 4-stage
// LDS ring of 128 x 64 bf16 A tiles (16 KB each), one barrier per k-step, and
// per wave and step 16 MFMAs (4 row tiles x 4 sub-steps of 16 k) on A
// fragments read from the step's stage and a fixed B.  The A tiles come from
// a 4 MiB buffer (block b, step s: tile (7 b + s) mod 256), which the L2 and
// the Infinity Cache hold:
//   MODE 0: no A loads (the ring holds what the first steps left);
//   MODE 1: global_load_lds_dwordx4 straight into the stage 3 steps ahead,
//           waited for with vmcnt before the step's barrier (as the library);
//   MODE 2: global_load_dwordx4 into registers 2 steps ahead, ds_write_b128
//           into the stage one step ahead.
constexpr int kTileElems = 128 * 64;
// s_waitcnt immediates (gfx9 encoding): vmcnt(vm) with lgkmcnt(0), and
// lgkmcnt(0) alone
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 0xF) | ((vm >> 4) << 14) | (0x7 << 4); }
constexpr int kWaitLgkm0 = waitcnt_vm_lgkm0(63);
constexpr int kSrcTiles = 256;  // 4 MiB of bf16

template <int MODE, int WM = 1>
__global__ __launch_bounds__(kThreads, 2) void ring_kernel(const uint16_t* __restrict__ src, float* out, int steps) {
  typedef __attribute__((address_space(3))) void* lds_ptr_t;
  typedef __attribute__((address_space(1))) void* glb_ptr_t;
  __shared__ __attribute__((aligned(16))) uint16_t st[4][kTileElems];
  const int tid = int(threadIdx.x), lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, lh = lane >> 5;
  f32x16 acc[4];
  for (int i = 0; i < 4; ++i) acc[i] = f32x16{};
  const u32x4 b = {0x3F803F80u, 0x3F803F80u ^ unsigned(lane << 15), 0x3F803F80u, 0x3F803F80u};
  for (int i = tid; i < 4 * kTileElems / 8; i += kThreads)
    reinterpret_cast<u32x4*>(&st[0][0])[i] = u32x4{0x3F803F80u, unsigned(i), 0x3F803F80u, 0u};
  __syncthreads();
  // element offset of this lane's 16 bytes in slot j of a tile, and of tile s
  auto lane_elem = [&](int j) { return (wave * 4 + j) * 512 + lane * 8; };
  auto tile_of = [&](int s) { return size_t((7 * int(blockIdx.x) + s) % kSrcTiles) * kTileElems; };
  auto dma = [&](int s) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_global_load_lds((glb_ptr_t)(src + tile_of(s) + lane_elem(j)),
                                       (lds_ptr_t)(&st[s & 3][(wave * 4 + j) * 512]), 16, 0, 0);
  };
  u32x4 reg[2][4];
  auto gload = [&](int s, u32x4 (&r)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = *reinterpret_cast<const u32x4*>(src + tile_of(s) + lane_elem(j));
  };
  auto gput = [&](int s, const u32x4 (&r)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4*>(&st[s & 3][lane_elem(j)]) = r[j];
  };
  if constexpr (MODE == 1) {
    dma(0);
    dma(1);
    dma(2);
  }
  if constexpr (MODE == 2) {
    gload(0, reg[0]);
    gload(1, reg[1]);
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) lgkmcnt(0): both register sets landed
    gput(0, reg[0]);
    gload(2, reg[0]);
  }
  // one k-step; step ks writes the registers of step ks + 1 (loaded two steps
  // before) into their stage and loads step ks + 3 into the same set
  auto step = [&](int ks, u32x4 (&r)[4]) {
    if constexpr (MODE == 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(8));  // fills ks + 1, ks + 2 in flight
    if constexpr (MODE == 2) {
      gput(ks + 1, r);
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if constexpr (MODE == 1) dma(ks + 3);
    if constexpr (MODE == 2) gload(ks + 3, r);
    const uint16_t* a = st[ks & 3];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // WM = 1: the wave's 4 row tiles, one MFMA each; WM = 2: 2 row tiles of
        // the wave's half of the rows, each A fragment feeding 2 MFMAs
        if (WM == 1 || i < 2) {
          const int r = (WM == 1 ? 0 : 64 * (wave >> 1)) + 32 * i + lr;  // library's chunk swizzle
          const u32x4 af = *reinterpret_cast<const u32x4*>(a + r * 64 + (((2 * s + lh) ^ ((r ^ (r >> 3)) & 7)) << 3));
#pragma unroll
          for (int u = 0; u < WM; ++u)
            acc[WM * i + u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af),
                                                                      __builtin_bit_cast(bf16x8, b), acc[WM * i + u],
                                                                      0, 0, 0);
        }
      }
  };
  for (int ks = 0; ks + 2 <= steps; ks += 2) {  // steps is even
    step(ks, reg[1]);
    step(ks + 1, reg[0]);
  }
  __builtin_amdgcn_s_waitcnt(0);
  float sum = 0.f;
  for (int i = 0; i < 4; ++i)
    for (int e = 0; e < 16; ++e) sum += acc[i][e];
  out[blockIdx.x * kThreads + tid] = sum;
}

bool ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return false;
}

// mean ms of 5 launches after one warm-up launch
template <typename K>
bool time_kernel(K kernel, float* out, int blocks, int iters, hipEvent_t a, hipEvent_t b, float& ms) {
  hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kThreads), 0, 0, out, iters);
  if (!ok(hipGetLastError(), "launch") || !ok(hipEventRecord(a), "event")) return false;
  for (int r = 0; r < 5; ++r) hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kThreads), 0, 0, out, iters);
  if (!ok(hipEventRecord(b), "event") || !ok(hipEventSynchronize(b), "sync")) return false;
  if (!ok(hipEventElapsedTime(&ms, a, b), "elapsed")) return false;
  ms /= 5;
  return true;
}

constexpr double kMfmaFlops = 32.0 * 32 * 16 * 2;

template <int V, bool DEP>
bool valu_case(float* out, int blocks, hipEvent_t a, hipEvent_t b) {
  const int iters = 2000;
  float ms = 0.f;
  if (!time_kernel(valu_kernel<V, DEP>, out, blocks, iters, a, b, ms)) return false;
  const double mfmas = double(blocks) * (kThreads / 64) * iters * 8;
  printf("{\"case\": \"valu\", \"valu_per_mfma\": %d, \"dependent\": %s, \"blocks\": %d, \"ms\": %.4f, "
         "\"tflops\": %.1f}\n",
         V, DEP ? "true" : "false", blocks, ms, mfmas * kMfmaFlops / (ms * 1e-3) / 1e12);
  fflush(stdout);
  return true;
}

template <int U>
bool lds_case(float* out, int blocks, hipEvent_t a, hipEvent_t b) {
  const int iters = U == 0 ? 4000 : 4000 / U;
  float ms = 0.f;
  if (!time_kernel(lds_kernel<U>, out, blocks, iters, a, b, ms)) return false;
  const double reads = double(blocks) * (kThreads / 64) * iters * 8;  // wave-wide 1 KB reads
  printf("{\"case\": \"lds\", \"mfma_per_fragment\": %d, \"blocks\": %d, \"ms\": %.4f, \"lds_bytes_per_clk_per_cu_at_2.4ghz\": "
         "%.1f, \"tflops\": %.1f}\n",
         U, blocks, ms, reads * 1024 / (ms * 1e-3) / 2.4e9 / 256, reads * U * kMfmaFlops / (ms * 1e-3) / 1e12);
  fflush(stdout);
  return true;
}

template <int MODE, int WM = 1>
bool ring_case(const uint16_t* src, float* out, int blocks, hipEvent_t a, hipEvent_t b) {
  const int steps = 2000;
  hipLaunchKernelGGL((ring_kernel<MODE, WM>), dim3(blocks), dim3(kThreads), 0, 0, src, out, steps);
  if (!ok(hipGetLastError(), "launch") || !ok(hipEventRecord(a), "event")) return false;
  for (int r = 0; r < 5; ++r)
    hipLaunchKernelGGL((ring_kernel<MODE, WM>), dim3(blocks), dim3(kThreads), 0, 0, src, out, steps);
  float ms = 0.f;
  if (!ok(hipEventRecord(b), "event") || !ok(hipEventSynchronize(b), "sync") || !ok(hipEventElapsedTime(&ms, a, b), "t"))
    return false;
  ms /= 5;
  const double mfmas = double(blocks) * (kThreads / 64) * steps * 16;
  printf("{\"case\": \"ring\", \"waves\": \"%s\", \"a_tiles\": \"%s\", \"blocks\": %d, \"ms\": %.4f, "
         "\"tflops\": %.1f}\n",
         WM == 1 ? "1x4 (4 x 1 tiles)" : "2x2 (2 x 2 tiles)",
         MODE == 0 ? "none" : MODE == 1 ? "global_load_lds" : "global_load + ds_write", blocks, ms,
         mfmas * kMfmaFlops / (ms * 1e-3) / 1e12);
  fflush(stdout);
  return true;
}

}  // namespace

int main() {
  float* out = nullptr;
  if (!ok(hipMalloc(&out, size_t(kMaxBlocks) * kThreads * sizeof(float)), "hipMalloc")) return 1;
  hipEvent_t a, b;
  if (!ok(hipEventCreate(&a), "event") || !ok(hipEventCreate(&b), "event")) return 1;
  bool good = true;
  uint16_t* src = nullptr;
  if (!ok(hipMalloc(&src, size_t(kSrcTiles) * kTileElems * sizeof(uint16_t)), "hipMalloc") ||
      !ok(hipMemset(src, 0x3F, size_t(kSrcTiles) * kTileElems * sizeof(uint16_t)), "hipMemset"))
    return 1;
  good = good && ring_case<0>(src, out, 512, a, b) && ring_case<1>(src, out, 512, a, b) &&
         ring_case<2>(src, out, 512, a, b) && ring_case<0, 2>(src, out, 512, a, b) &&
         ring_case<1, 2>(src, out, 512, a, b);
  good = good && valu_case<0, false>(out, 256, a, b) && valu_case<4, false>(out, 256, a, b) &&
         lds_case<1>(out, 256, a, b) && lds_case<2>(out, 256, a, b);  // one wave per SIMD
  for (int blocks : {512, kMaxBlocks}) {
    good = good && valu_case<0, false>(out, blocks, a, b) && valu_case<2, false>(out, blocks, a, b) &&
           valu_case<4, false>(out, blocks, a, b) && valu_case<6, false>(out, blocks, a, b) &&
           valu_case<8, false>(out, blocks, a, b) && valu_case<12, false>(out, blocks, a, b) &&
           valu_case<4, true>(out, blocks, a, b) && valu_case<8, true>(out, blocks, a, b);
    good = good && lds_case<0>(out, blocks, a, b) && lds_case<1>(out, blocks, a, b) &&
           lds_case<2>(out, blocks, a, b) && lds_case<4>(out, blocks, a, b);
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  (void)hipFree(out);
  (void)hipFree(src);
  return good ? 0 : 1;
}
