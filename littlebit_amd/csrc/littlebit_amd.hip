// LittleBitLinear forward for MI355X (gfx950): kernels and the C ABI of
// include/littlebit_amd.h.
//
// The forward of one projection is
//     y[m, n] = bias[n] + sum_b h_b[n] * sum_r sU_b[n, r] * t_b[m, r]
//     t_b[m, r] = l_b[r] * sum_k sV_b[r, k] * g_b[k] * x[m, k]
// (quantization/modules/littlebit.py:95-121 with g = v2, l = v1*u2, h = u1),
// where sV and sU are +-1 read from words packed LSB first, bit 1 == -1
// (quantization/utils/binary_packer.py:36-50).
//
// Two launches per projection, both branches in each:
//   latent_kernel : one wavefront per latent row r of every branch; lanes
//                   stride over the row's words, the wave reduces, lane 0
//                   writes t[m, r] (already multiplied by l[r]) to workspace.
//   expand_kernel : t of both branches staged in LDS; LPR lanes per output
//                   row n split the row's words, reduce with lane shuffles and
//                   write h0*acc0 + h1*acc1 + bias.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "littlebit_amd.h"

namespace {

thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int64_t kMaxDim = int64_t(1) << 24;     // K, N, M limit
constexpr int64_t kMaxRankTotal = 16384;          // sum of branch ranks
constexpr int kLdsBudget = 64 * 1024;             // t staging in expand_kernel

struct DevBranch {
  const uint32_t* v;  // [R, KW]
  const uint32_t* u;  // [N, RW]
  const float* g;     // [K]
  const float* l;     // [R]
  const float* h;     // [N]
  float* t;           // workspace [M, R], l-scaled latent
  int R;
  int RW;
  int block0;         // first latent_kernel block of this branch
};

struct FwdParams {
  DevBranch br[2];
  int nb;
  int M, K, KW, N;
  const void* x;
  const float* bias;
  void* y;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(uint16_t v) {
  return __uint_as_float(uint32_t(v) << 16);
}

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

__device__ __forceinline__ void store_out(float* y, size_t i, float v) { y[i] = v; }
__device__ __forceinline__ void store_out(uint16_t* y, size_t i, float v) {
  y[i] = f32_to_bf16(v);
}

__device__ __forceinline__ DevBranch pick(const FwdParams& p, int b) {
  return b ? p.br[1] : p.br[0];
}

// ---------------------------------------------------------------------------
// Stage 1: t[m, r] = l[r] * sum_k sV[r, k] * g[k] * x[m, k]
// grid.x = sum_b ceil(R_b / 4) (one wave per row), grid.y = ceil(M / MT)
// ---------------------------------------------------------------------------
template <typename XT, int MT>
__global__ __launch_bounds__(kBlock) void latent_kernel(FwdParams p) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int b = (p.nb > 1 && int(blockIdx.x) >= p.br[1].block0) ? 1 : 0;
  const DevBranch B = pick(p, b);
  const int r = (int(blockIdx.x) - B.block0) * kWavesPerBlock + wave;
  if (r >= B.R) return;  // uniform per wave
  const int m0 = int(blockIdx.y) * MT;
  const XT* x = static_cast<const XT*>(p.x);

  float acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = 0.f;

  const uint32_t* vrow = B.v + size_t(r) * p.KW;
  for (int w = lane; w < p.KW; w += kWave) {
    const uint32_t bits = vrow[w];
    const int k0 = w * 32;
    const int kn = min(32, p.K - k0);
    for (int j = 0; j < kn; ++j) {
      const float gk = B.g[k0 + j];
      const bool neg = (bits >> j) & 1u;
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int m = m0 + i;
        if (m < p.M) {
          const float a = gk * to_f32(x[size_t(m) * p.K + k0 + j]);
          acc[i] += neg ? -a : a;
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    float v = acc[i];
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    acc[i] = v;
  }
  if (lane == 0) {
    const float lr = B.l[r];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int m = m0 + i;
      if (m < p.M) B.t[size_t(m) * B.R + r] = lr * acc[i];
    }
  }
}

// ---------------------------------------------------------------------------
// Stage 2: y[m, n] = bias[n] + sum_b h_b[n] * sum_r sU_b[n, r] * t_b[m, r]
// grid.x = ceil(N / (256 / LPR)), grid.y = ceil(M / MT); LDS holds t.
// ---------------------------------------------------------------------------
template <typename YT, int MT, int LPR>
__global__ __launch_bounds__(kBlock) void expand_kernel(FwdParams p) {
  extern __shared__ float lds_t[];  // per branch [MT][R_b]
  const int m0 = int(blockIdx.y) * MT;

  int off = 0;
  for (int b = 0; b < p.nb; ++b) {
    const DevBranch B = pick(p, b);
    for (int i = threadIdx.x; i < MT * B.R; i += kBlock) {
      const int mi = i / B.R;
      const int r = i - mi * B.R;
      const int m = m0 + mi;
      lds_t[off + i] = (m < p.M) ? B.t[size_t(m) * B.R + r] : 0.f;
    }
    off += MT * B.R;
  }
  __syncthreads();

  const int n = int(blockIdx.x) * (kBlock / LPR) + int(threadIdx.x) / LPR;
  const int q = int(threadIdx.x) % LPR;
  float out[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) out[i] = 0.f;

  off = 0;
  for (int b = 0; b < p.nb; ++b) {
    const DevBranch B = pick(p, b);
    float acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = 0.f;
    if (n < p.N) {
      const uint32_t* urow = B.u + size_t(n) * B.RW;
      for (int w = q; w < B.RW; w += LPR) {
        const uint32_t bits = urow[w];
        const int r0 = w * 32;
        const int rn = min(32, B.R - r0);
        for (int j = 0; j < rn; ++j) {
          const bool neg = (bits >> j) & 1u;
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            const float tv = lds_t[off + i * B.R + r0 + j];
            acc[i] += neg ? -tv : tv;
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      float v = acc[i];
#pragma unroll
      for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
      acc[i] = v;
    }
    const float hn = (n < p.N) ? B.h[n] : 0.f;
#pragma unroll
    for (int i = 0; i < MT; ++i) out[i] += hn * acc[i];
    off += MT * B.R;
  }

  if (n < p.N && q == 0) {
    const float bn = p.bias ? p.bias[n] : 0.f;
    YT* y = static_cast<YT*>(p.y);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int m = m0 + i;
      if (m < p.M) store_out(y, size_t(m) * p.N + n, out[i] + bn);
    }
  }
}

// ---------------------------------------------------------------------------
// Sign pack / unpack (bit-exact with the reference packer)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void unpack_kernel(const uint32_t* packed, int64_t rows,
                                                        int64_t cols, int64_t wpr, int8_t* out) {
  const int64_t total = rows * cols;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * kBlock) {
    const int64_t r = i / cols;
    const int64_t c = i - r * cols;
    const uint32_t word = packed[r * wpr + (c >> 5)];
    out[i] = int8_t(1 - 2 * int((word >> (c & 31)) & 1u));
  }
}

__global__ __launch_bounds__(kBlock) void pack_kernel(const int8_t* signs, int64_t rows,
                                                      int64_t cols, int64_t wpr, uint32_t* out) {
  const int64_t total = rows * wpr;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * kBlock) {
    const int64_t r = i / wpr;
    const int64_t w = i - r * wpr;
    const int64_t c0 = w * 32;
    const int cn = int(cols - c0 < 32 ? cols - c0 : 32);
    const int8_t* row = signs + r * cols + c0;
    uint32_t word = 0;
    for (int j = 0; j < cn; ++j) word |= uint32_t(row[j] < 0) << j;
    out[i] = word;
  }
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(LBK_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return LBK_OK;
}

int validate(const lbk_branch* branches, int n_branches, int64_t M, int64_t K, int64_t N) {
  if (!branches) return set_error(LBK_ERR_ARG, "branches is NULL");
  if (n_branches < 1 || n_branches > 2)
    return set_error(LBK_ERR_ARG, "n_branches must be 1 or 2, got %d", n_branches);
  if (M < 0 || M > kMaxDim) return set_error(LBK_ERR_ARG, "M must be in [0, %lld], got %lld", (long long)kMaxDim, (long long)M);
  if (K < 1 || K > kMaxDim) return set_error(LBK_ERR_ARG, "K must be in [1, %lld], got %lld", (long long)kMaxDim, (long long)K);
  if (N < 1 || N > kMaxDim) return set_error(LBK_ERR_ARG, "N must be in [1, %lld], got %lld", (long long)kMaxDim, (long long)N);
  int64_t rsum = 0;
  for (int b = 0; b < n_branches; ++b) {
    const lbk_branch& B = branches[b];
    if (B.rank < 1) return set_error(LBK_ERR_ARG, "branch %d: rank must be >= 1, got %lld", b, (long long)B.rank);
    if (!B.v_sign || !B.u_sign || !B.v2 || !B.mid || !B.u1)
      return set_error(LBK_ERR_ARG, "branch %d: NULL factor or scale pointer", b);
    rsum += B.rank;
  }
  if (rsum > kMaxRankTotal)
    return set_error(LBK_ERR_ARG, "sum of branch ranks %lld exceeds %lld", (long long)rsum, (long long)kMaxRankTotal);
  return LBK_OK;
}

size_t workspace_for(const lbk_branch* branches, int n_branches, int64_t M) {
  size_t bytes = 0;
  for (int b = 0; b < n_branches; ++b) bytes += align256(size_t(M) * size_t(branches[b].rank) * sizeof(float));
  return bytes;
}

template <typename XT>
void launch_latent(const FwdParams& p, int mt, dim3 grid, hipStream_t s) {
  switch (mt) {
    case 1: hipLaunchKernelGGL((latent_kernel<XT, 1>), grid, dim3(kBlock), 0, s, p); break;
    case 2: hipLaunchKernelGGL((latent_kernel<XT, 2>), grid, dim3(kBlock), 0, s, p); break;
    case 4: hipLaunchKernelGGL((latent_kernel<XT, 4>), grid, dim3(kBlock), 0, s, p); break;
    default: hipLaunchKernelGGL((latent_kernel<XT, 8>), grid, dim3(kBlock), 0, s, p); break;
  }
}

template <typename YT, int MT>
void launch_expand_lpr(const FwdParams& p, int lpr, size_t lds, hipStream_t s) {
  const int rows = kBlock / lpr;
  const dim3 grid{unsigned(ceil_div(p.N, rows)), unsigned(ceil_div(p.M, MT)), 1u};
  switch (lpr) {
    case 4: hipLaunchKernelGGL((expand_kernel<YT, MT, 4>), grid, dim3(kBlock), lds, s, p); break;
    case 16: hipLaunchKernelGGL((expand_kernel<YT, MT, 16>), grid, dim3(kBlock), lds, s, p); break;
    default: hipLaunchKernelGGL((expand_kernel<YT, MT, 64>), grid, dim3(kBlock), lds, s, p); break;
  }
}

template <typename YT>
void launch_expand(const FwdParams& p, int mt, int lpr, size_t lds, hipStream_t s) {
  switch (mt) {
    case 1: launch_expand_lpr<YT, 1>(p, lpr, lds, s); break;
    case 2: launch_expand_lpr<YT, 2>(p, lpr, lds, s); break;
    case 4: launch_expand_lpr<YT, 4>(p, lpr, lds, s); break;
    default: launch_expand_lpr<YT, 8>(p, lpr, lds, s); break;
  }
}

int mtile_for(int64_t M, int64_t cap) {
  int mt = 8;
  while (mt > 1 && (mt > cap || (mt / 2) >= M)) mt /= 2;
  return mt;
}

}  // namespace

extern "C" {

int lbk_abi_version(void) { return LBK_ABI_VERSION; }

const char* lbk_last_error(void) { return g_last_error; }

size_t lbk_linear_workspace_bytes(const lbk_branch* branches, int n_branches, int64_t M, int64_t K,
                                  int64_t N) {
  if (validate(branches, n_branches, M, K, N) != LBK_OK) return 0;
  return workspace_for(branches, n_branches, M);
}

int lbk_linear_forward(const lbk_branch* branches, int n_branches, int64_t M, int64_t K, int64_t N,
                       const void* x, int x_dtype, const float* bias, void* y, int y_dtype,
                       void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error[0] = '\0';
  int rc = validate(branches, n_branches, M, K, N);
  if (rc != LBK_OK) return rc;
  if (x_dtype != LBK_F32 && x_dtype != LBK_BF16) return set_error(LBK_ERR_DTYPE, "x_dtype %d unsupported", x_dtype);
  if (y_dtype != LBK_F32 && y_dtype != LBK_BF16) return set_error(LBK_ERR_DTYPE, "y_dtype %d unsupported", y_dtype);
  if (M == 0) return LBK_OK;
  if (!x || !y) return set_error(LBK_ERR_ARG, "x or y is NULL");
  const size_t need = workspace_for(branches, n_branches, M);
  if (!workspace || workspace_bytes < need)
    return set_error(LBK_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);

  FwdParams p;
  memset(&p, 0, sizeof(p));
  p.nb = n_branches;
  p.M = int(M);
  p.K = int(K);
  p.KW = int(ceil_div(K, 32));
  p.N = int(N);
  p.x = x;
  p.bias = bias;
  p.y = y;
  char* ws = static_cast<char*>(workspace);
  int blocks = 0;
  int64_t rsum = 0;
  int rw_max = 0;
  for (int b = 0; b < n_branches; ++b) {
    const lbk_branch& S = branches[b];
    DevBranch& D = p.br[b];
    D.v = reinterpret_cast<const uint32_t*>(S.v_sign);
    D.u = reinterpret_cast<const uint32_t*>(S.u_sign);
    D.g = S.v2;
    D.l = S.mid;
    D.h = S.u1;
    D.R = int(S.rank);
    D.RW = int(ceil_div(S.rank, 32));
    D.t = reinterpret_cast<float*>(ws);
    ws += align256(size_t(M) * size_t(S.rank) * sizeof(float));
    D.block0 = blocks;
    blocks += int(ceil_div(S.rank, kWavesPerBlock));
    rsum += S.rank;
    if (D.RW > rw_max) rw_max = D.RW;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);

  const int mt1 = mtile_for(M, 8);
  const int64_t mchunks1 = ceil_div(M, mt1);
  if (mchunks1 > 65535) return set_error(LBK_ERR_ARG, "M=%lld too large for this path", (long long)M);
  const dim3 g1{unsigned(blocks), unsigned(mchunks1), 1u};
  if (x_dtype == LBK_F32) launch_latent<float>(p, mt1, g1, s);
  else launch_latent<uint16_t>(p, mt1, g1, s);
  rc = check_launch("latent_kernel");
  if (rc != LBK_OK) return rc;

  const int64_t cap = kLdsBudget / (rsum * int64_t(sizeof(float)));
  const int mt2 = mtile_for(M, cap < 1 ? 1 : cap);
  if (ceil_div(M, mt2) > 65535) return set_error(LBK_ERR_ARG, "M=%lld too large for this path", (long long)M);
  const size_t lds = size_t(rsum) * mt2 * sizeof(float);
  const int lpr = rw_max <= 8 ? 4 : (rw_max <= 32 ? 16 : 64);
  if (y_dtype == LBK_F32) launch_expand<float>(p, mt2, lpr, lds, s);
  else launch_expand<uint16_t>(p, mt2, lpr, lds, s);
  return check_launch("expand_kernel");
}

int lbk_littlebit_linear(const float* input, int64_t M, const float* v2, const int32_t* v_sign,
                         int64_t v_cols, const float* mid, const int32_t* u_sign, int64_t u_cols,
                         const float* u1, int64_t out_features, float* output, void* workspace,
                         size_t workspace_bytes, void* stream) {
  lbk_branch b;
  b.v_sign = v_sign;
  b.u_sign = u_sign;
  b.v2 = v2;
  b.mid = mid;
  b.u1 = u1;
  b.rank = u_cols;
  return lbk_linear_forward(&b, 1, M, v_cols, out_features, input, LBK_F32, nullptr, output, LBK_F32,
                            workspace, workspace_bytes, stream);
}

int lbk_unpack_signs(const int32_t* packed, int64_t rows, int64_t cols, int8_t* out, void* stream) {
  g_last_error[0] = '\0';
  if (rows < 0 || cols < 0) return set_error(LBK_ERR_ARG, "negative shape");
  if (rows == 0 || cols == 0) return LBK_OK;
  if (!packed || !out) return set_error(LBK_ERR_ARG, "NULL pointer");
  const int64_t total = rows * cols;
  const int64_t blocks = ceil_div(total, kBlock) < 65536 ? ceil_div(total, kBlock) : 65536;
  hipLaunchKernelGGL(unpack_kernel, dim3(unsigned(blocks)), dim3(kBlock), 0, static_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint32_t*>(packed), rows, cols, ceil_div(cols, 32), out);
  return check_launch("unpack_kernel");
}

int lbk_pack_signs(const int8_t* signs, int64_t rows, int64_t cols, int32_t* out, void* stream) {
  g_last_error[0] = '\0';
  if (rows < 0 || cols < 0) return set_error(LBK_ERR_ARG, "negative shape");
  if (rows == 0 || cols == 0) return LBK_OK;
  if (!signs || !out) return set_error(LBK_ERR_ARG, "NULL pointer");
  const int64_t wpr = ceil_div(cols, 32);
  const int64_t total = rows * wpr;
  const int64_t blocks = ceil_div(total, kBlock) < 65536 ? ceil_div(total, kBlock) : 65536;
  hipLaunchKernelGGL(pack_kernel, dim3(unsigned(blocks)), dim3(kBlock), 0, static_cast<hipStream_t>(stream),
                     signs, rows, cols, wpr, reinterpret_cast<uint32_t*>(out));
  return check_launch("pack_kernel");
}

}  // extern "C"
