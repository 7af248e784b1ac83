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
// Two launches per call, every branch in each; a call covers one projection
// or a group of up to four projections that read the same x (q/k/v, gate/up).
//
// MFMA path (M <= 8 in one pass; 9-64 rows as 8-row chunks side by side in
// one launch pair, chunk = grid.y of the latent kernel, grid.z of the expand
// kernel; deterministic mode takes 9-16 rows in one 16-row pass):
//   latent_mfma_kernel  grid = row-blocks (64 latent rows of one branch) x
//                       k-chunks.  The block writes bf16 hi/lo halves of
//                       g*x for its k-chunk to LDS (the MFMA A operand: rows
//                       0-7 = hi of m 0-7, rows 8-15 = lo); each wave expands
//                       its 16 rows' sign bytes into +-1 bf16 B operands in
//                       registers and runs v_mfma_f32_16x16x32_bf16.  The
//                       k-chunks add l-scaled partial sums into the latent
//                       buffer t with fp32 atomics.
//   expand_mfma_kernel  grid = (16-row tiles of a projection per block, rank
//                       slices).  The t chunks of the block's slice of the
//                       projection's branches are staged in LDS as bf16
//                       hi/lo; each wave expands the U sign bytes of its 16
//                       rows and accumulates both branches, then writes
//                       h0*y0 + h1*y1 + bias (one slice) or adds h0*y0 +
//                       h1*y1 to y with fp32 atomics (several slices; the
//                       latent kernel has set y = bias + residual).
// GEMM path (M > 64, or operands too large for the decode path's LDS):
//   gemm_scale_kernel (bf16 g*x, when x cannot be read as it is) /
//   gemm_latent_kernel (or its stream-K form) / gemm_expand_kernel (or its
//   128 x 256 tile form), tiled on v_mfma_f32_32x32x16_bf16.
//
// Splitting fp32 activations into bf16 hi + lo keeps the product error near
// 2^-17 relative: +-1 is exact in bf16 and the MFMA accumulates in fp32.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <climits>
#include <atomic>
#include <mutex>
#include <type_traits>

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
constexpr int64_t kMaxDim = int64_t(1) << 24;  // K, N, M limit
constexpr int64_t kMaxRankTotal = 16384;       // sum of branch ranks
constexpr int kLdsPerCU = 160 * 1024;          // gfx950: LDS per CU
constexpr int kMaxBlockLds = 159 * 1024;       // static + dynamic LDS of one block (a 160 KB request failed to launch)
constexpr int kRowBlock = 64;                  // latent rows per latent_mfma block
constexpr int kMaxMfmaM = 16;                  // MFMA path handles M <= 16
constexpr int kCounterSlots = 1024;            // counters at the workspace start
constexpr float kTinyH = 1e-30f;               // |h1| below this: no h0 / h1 rescale (it could overflow)
constexpr float kMaxHRatio = 1099511627776.f;  // 2^40: |h0 / h1| above this drops branch 1 (wide stage 2)
constexpr size_t kCounterBytes = kCounterSlots * sizeof(uint32_t);

// Encoding of s_waitcnt vmcnt(n) lgkmcnt(0) on gfx9 (expcnt left alone).
constexpr int waitcnt_vm_lgkm0(int n) { return (n & 15) | (7 << 4) | ((n >> 4) << 14); }

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// element helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }

// fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// Wide stage 2 keeps branch 1 of a column (rescaling acc by h0 / h1) unless
// h1 is zero or denormal, or |h0 / h1| > 2^40 (the rescaled acc could
// overflow, while h1's term is negligible there).
__device__ __forceinline__ bool use_branch1(float h0, float h1) {
  return fabsf(h1) >= kTinyH && fabsf(h0) <= fabsf(h1) * kMaxHRatio;
}

__device__ __forceinline__ void store_out(float* y, size_t i, float v) { y[i] = v; }
__device__ __forceinline__ void store_out(uint16_t* y, size_t i, float v) { y[i] = f32_to_bf16(v); }


// 8 consecutive floats from a 16-byte aligned address.
__device__ __forceinline__ void load8(const float* p, float (&a)[8]) {
  const float4 u = *reinterpret_cast<const float4*>(p);
  const float4 w = *reinterpret_cast<const float4*>(p + 4);
  a[0] = u.x; a[1] = u.y; a[2] = u.z; a[3] = u.w;
  a[4] = w.x; a[5] = w.y; a[6] = w.z; a[7] = w.w;
}
// 8 consecutive bf16 (as raw bits) from a 16-byte aligned address.
__device__ __forceinline__ void load8(const uint16_t* p, float (&a)[8]) {
  const u32x4 u = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    a[2 * d] = __uint_as_float(u[d] << 16);
    a[2 * d + 1] = __uint_as_float(u[d] & 0xffff0000u);
  }
}

// 8 consecutive elements from a 16-byte aligned address, kept as loaded and
// converted to float only by get(): a batch of Raw8 loads is issued before
// any of it is waited for.
template <typename T>
struct Raw8;
template <>
struct Raw8<float> {
  float4 u, w;
  __device__ __forceinline__ void load(const float* p) {
    u = *reinterpret_cast<const float4*>(p);
    w = *reinterpret_cast<const float4*>(p + 4);
  }
  __device__ __forceinline__ void get(float (&a)[8]) const {
    a[0] = u.x; a[1] = u.y; a[2] = u.z; a[3] = u.w;
    a[4] = w.x; a[5] = w.y; a[6] = w.z; a[7] = w.w;
  }
};
template <>
struct Raw8<uint16_t> {
  u32x4 u;
  __device__ __forceinline__ void load(const uint16_t* p) { u = *reinterpret_cast<const u32x4*>(p); }
  __device__ __forceinline__ void get(float (&a)[8]) const {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      a[2 * d] = __uint_as_float(u[d] << 16);
      a[2 * d + 1] = __uint_as_float(u[d] & 0xffff0000u);
    }
  }
};

// ---------------------------------------------------------------------------
// MFMA path parameters
// ---------------------------------------------------------------------------
constexpr int kMaxWaveSteps = 32;  // rank steps (both branches) per expand wave
// positions per wave of the decode attention (16 measured faster at KV 512
// than 8 or 32); its partials are rows of head_dim + kAttnPad floats (o, then
// max and exp-sum, 16-byte aligned rows)
constexpr int kAttnChunk = 16;
constexpr int kAttnPad = 4;
constexpr int kMaxProj = 4;        // projections sharing one input in a group call
constexpr int kMaxSeg = 2 * kMaxProj;
// floats per latent half: M <= 16 rows of the padded ranks of every branch,
// then kSsqSlots sums of squares (one per row of a call whose row chunks run
// in one launch pair, up to 64 rows when t fits)
constexpr int kSsqSlots = 64;
constexpr int kTHalf = kMaxMfmaM * (kMaxRankTotal + kMaxSeg * 128) + kSsqSlots;
// t of a call pads each branch's rank by less than 128, so 16 rows and the
// sums of squares after them always fit
static_assert(kMaxMfmaM * (kMaxRankTotal + kMaxSeg * 127) + kSsqSlots <= kTHalf, "latent half too small");
static_assert(kTHalf % 4 == 0, "latent halves are read in float4s");

// Stage-1 operands of one branch ("segment") of a group call.
struct LatSeg {
  const uint32_t* V;  // [R, KW] sign words
  const uint32_t* Vt; // the same words tiled (see tile_v_kernel), or null
  const float* g;     // [K]
  const float* l;     // [R]
  int R;
  int RP;     // padded latent row length (multiple of 128)
  int rb0;    // first row-block of the segment
  int tbase;  // offset of the segment's [M][RP] block in t
};

// Stage-2 operands of one projection (one or two segments) of a group call.
struct ExpProj {
  const uint32_t* U[2];  // [N, RW] sign words per branch
  const float* h[2];     // [N]
  const float* bias;     // [N] or null
  const float* res;      // [M, N] fp32 added to y, or null (may alias y)
  void* y;               // [M, N]
  int RW[2];    // words per U row
  int RWp[2];   // RW rounded up to a multiple of 4
  int RP[2];    // 32 * RWp
  int tbase[2];
  int nb;
  int N;
  int tile0;    // first expand block of the projection
};

struct MfmaParams {
  LatSeg seg[kMaxSeg];
  ExpProj proj[kMaxProj];
  int nseg, nproj;
  int M, K, KW;
  int crows;    // rows per row chunk: chunk c (latent grid.y, expand grid.z) takes rows
                // [c * crows, min(M, (c + 1) * crows)); crows = M with one chunk
  int tsize;    // M * sum(RP) floats
  int nkc;      // k-chunks
  int kc_major; // latent blocks in k-chunk-major order (every segment reads V's tiled copy)
  int splits;   // expand_mfma_kernel: waves sharing the rank steps of a 16-row tile
  int ntiles;   // expand_mfma_kernel: row tiles of all projections (grid.x may be padded)
  int ks;       // expand_mfma_kernel: rank slices per projection (grid.y); with ks > 1
                // the latent kernel sets y = bias + residual and the slices add
                // their parts with fp32 atomics (fp32 y not overlapping x only)
  int xvec;     // x (x1, rms weight) and every g allow 16-byte loads (aligned, K % 8 == 0)
  int wvec;     // V rows allow WPL-word vector loads (16-byte aligned rows, KW % max(WPL, 4) == 0)
  int xmode;    // LBK_INPUT_*: x as is, RMSNorm(x) * w, or SiLU(x) * x1
  int late_rs;  // RMSNorm input staged without 1/rms: expand_mfma_kernel scales t
  const void* x;
  const void* x1;       // second input of LBK_INPUT_SILU_MUL
  const float* nw;      // RMSNorm weight [K]
  float eps;            // RMSNorm epsilon
  // LBK_INPUT_ATTN_MERGE: x = attention partials [K / ahd][achunks][ahd + 4];
  // position from apos when set, else apos_host
  const int64_t* apos;
  int64_t apos_host;
  int ahd, achunks, amax_seq;
  float* t2;       // two halves of kTHalf floats; per segment [M][RP] latent, l-scaled,
                   // then kMaxMfmaM floats: per row the sum of x^2 (RMSNorm input)
  uint32_t* sync;  // [0] P: half the next latent kernel accumulates into
                   // [1] Q: half the last latent kernel accumulated into
                   // [2 + h] floats of half h that may be non-zero
  // Deterministic mode with nkc > 1: the k-chunks store their partial t in
  // part[kc][tsize] and the sums of squares in part[nkc * tsize + (2 kc +
  // sub) * kMaxMfmaM + m] (sub: the second wave of a 128-chunk row group);
  // the last block of a row-block to finish (counted in det_cnt[row-block],
  // zero between calls) sums its rows' partials in chunk order into the
  // half.  Null otherwise (partials meet in fp32 atomics, in no fixed order).
  float* part;
  uint32_t* det_cnt;
  // Chains (one row, see chain_mfma_kernel): explicit latent regions instead
  // of the halves.  tdst set: the latent kernel accumulates t (and the sums
  // of squares at tdst + tsize) there and leaves the halves' state alone;
  // tsrc set: the expand kernel reads t there and leaves the state alone.
  // Either kernel then clears clr[0, nclr), spread over its blocks.
  float* tdst;
  const float* tsrc;
  float* clr;
  int nclr;
};

// Latent buffer protocol (all writes idempotent, so no ordering between
// blocks is needed; kernel boundaries order the rest):
//   latent_mfma_kernel: h = P; accumulate into half h (which is zero);
//     clear the first S[1-h] floats of half 1-h (making it all zero);
//     block 0 writes Q = h and S[h] = tsize + kMaxMfmaM (t, then the rows'
//     sums of squares of an RMSNorm input, added by the first row-block).
//   expand_mfma_kernel: reads t from half Q; block 0 writes P = 1 - Q.
// Calls of any shape may follow each other on one workspace; graph replay
// works because the state lives in device memory, not in kernel arguments.

// (x & m) | o, one v_and_or_b32.  That is VOP3, which takes no literal
// operands on gfx9, so the callers keep the masks in VGPRs (pinned by an
// empty asm so they are not re-materialised).  It must stay plain C: the
// result feeds an MFMA, and the compiler inserts the wait states between a
// VALU write and an MFMA read of the same register only for writes it can
// see -- the same instruction written as inline asm let MFMAs read stale B
// operands on gfx950 whenever the scheduler placed it right before them.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) { return (x & m) | o; }

// Byte j of a sign word -> 8 bf16 (+1 for bit 0, -1 for bit 1); element i is
// bit 8j+i.  Each dword holds elements 2d (low half) and 2d+1 (high half):
// the byte is replicated into both halves (one v_mul_u32_u24 with a byte
// select), a packed 16-bit shift moves bit 2d / 2d+1 to bit 15 of its half,
// and (x & 0x80008000) | 0x3F803F80 makes +-1.0: 9 VALU for 8 signs.
__device__ __forceinline__ bf16x8 signs_to_bf16x8(uint32_t word, int j, uint32_t kmask, uint32_t kone) {
  const uint32_t b = (word >> (8 * j)) & 0xffu;
  const uint32_t rep = b * 0x10001u;
  const u16x2 v = __builtin_bit_cast(u16x2, rep);
  u32x4 out;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const u16x2 sh = {(unsigned short)(15 - 2 * d), (unsigned short)(14 - 2 * d)};
    const u16x2 r = v << sh;
    out[d] = and_or(__builtin_bit_cast(uint32_t, r), kmask, kone);
  }
  return __builtin_bit_cast(bf16x8, out);
}

// Byte j of `word` times 8 bf16 values gv (two per dword, element order):
// bit i set flips the sign of element i (the +-1 of signs_to_bf16x8 times gv).
__device__ __forceinline__ bf16x8 signs_times_bf16x8(uint32_t word, int j, uint32_t kmask, u32x4 gv) {
  const uint32_t b = (word >> (8 * j)) & 0xffu;
  const uint32_t rep = b * 0x10001u;
  const u16x2 v = __builtin_bit_cast(u16x2, rep);
  u32x4 out;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const u16x2 sh = {(unsigned short)(15 - 2 * d), (unsigned short)(14 - 2 * d)};
    const u16x2 r = v << sh;
    out[d] = (__builtin_bit_cast(uint32_t, r) & kmask) ^ gv[d];
  }
  return __builtin_bit_cast(bf16x8, out);
}

// hi = bf16(a), lo = bf16(a - hi) of 8 floats, two per dword in element order
// (v_cvt_pk_bf16_f32, round to nearest even).
__device__ __forceinline__ void split8(const float (&a)[8], u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const f32x2 x = {a[2 * d], a[2 * d + 1]};
    const bf16x2 h = __builtin_convertvector(x, bf16x2);
    const f32x2 r = x - __builtin_convertvector(h, f32x2);
    hi[d] = __builtin_bit_cast(uint32_t, h);
    lo[d] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2));
  }
}

// x of lane l plus x of lane l + 32, in lanes 0..31 (lanes 32..63 get 2x;
// every caller reads the lower half only): MFMA C rows 0..7 (lanes 0..31)
// and 8..15 (lanes 32..63) hold the hi and lo parts of the same sums.
// v_permlane32_swap moves the upper half down in one VALU op; a shuffle
// through ds_bpermute costs an LDS round trip and a wait.
__device__ __forceinline__ float add_upper32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return x + __uint_as_float(r[1]);
}

// Sum over each row of 16 lanes, in every lane of the row: four DPP adds
// (quad swaps 1 and 2, then the half-row and row mirrors).
__device__ __forceinline__ float row16_sum(float s) {
  s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0xb1, 0xf, 0xf, false));
  s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x4e, 0xf, 0xf, false));
  s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x141, 0xf, 0xf, false));
  s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x140, 0xf, 0xf, false));
  return s;
}

// The same for W = 4 or 8 floats, as W / 2 dwords each.
template <int W>
__device__ __forceinline__ void split_pairs(const float (&a)[W], uint32_t (&hi)[W / 2], uint32_t (&lo)[W / 2]) {
#pragma unroll
  for (int d = 0; d < W / 2; ++d) {
    const f32x2 x = {a[2 * d], a[2 * d + 1]};
    const bf16x2 h = __builtin_convertvector(x, bf16x2);
    const f32x2 r = x - __builtin_convertvector(h, f32x2);
    hi[d] = __builtin_bit_cast(uint32_t, h);
    lo[d] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2));
  }
}
// N = 2 or 4 dwords to an 8- or 16-byte aligned LDS address, one store.
template <int N>
__device__ __forceinline__ void store_dwords(uint32_t* p, const uint32_t (&d)[N]) {
  if constexpr (N == 4) *reinterpret_cast<u32x4*>(p) = u32x4{d[0], d[1], d[2], d[3]};
  else *reinterpret_cast<u32x2*>(p) = u32x2{d[0], d[1]};
}

// An MFMA A operand in LDS, compact: for each m-block (8 m), each chunk of
// 8 k holds ROWS = 2*MR + 1 rows of 16 bytes: the hi halves of the MR
// stored m, their lo halves, and one zero row.  MFMA lane rows (0-7 hi,
// 8-15 lo of m = 0..7) that have no stored m read the zero row, so M = 1
// keeps 3 rows per chunk instead of 16.  Rows of M <= m < MT hold zeros.
template <int MT>
struct Compact {
  static constexpr int MB = (MT + 7) / 8;     // m-blocks
  static constexpr int MR = MT < 8 ? MT : 8;  // stored m per block
  static constexpr int ROWS = 2 * MR + 1;
  // row of MFMA lane row `col` (0..15) within a chunk
  __device__ static int lane_row(int col) {
    const int ml = col & 7;
    return ml < MR ? (col < 8 ? ml : MR + ml) : 2 * MR;
  }
};

// The effective input of a call, element (m, k) times g[k]:
//   LBK_INPUT_PLAIN     x[m, k]
//   LBK_INPUT_RMSNORM   x[m, k] * rs[m] * w[k],  rs[m] = 1 / sqrt(mean_k x[m, k]^2 + eps)
//   LBK_INPUT_SILU_MUL  x[m, k] / (1 + exp(-x[m, k])) * x1[m, k]
// (the RMSNorm, SiLU * up and their order are those of the reference's CPU
// decode step, patches/littlebit_cpu_optimized.cpp:1370-1438).
// SiLU with the hardware exp and reciprocal (v_exp_f32, v_rcp_f32: about 1
// ulp each).  An IEEE divide costs ~10 instructions, and the latent kernel
// evaluates SiLU for its whole k-chunk in every row-block.
__device__ __forceinline__ float silu_f(float v) { return v * __builtin_amdgcn_rcpf(1.f + __expf(-v)); }
// 1 / sqrt(ssum / K + eps) with v_rsq_f32 (about 1 ulp), kinv = 1 / K
__device__ __forceinline__ float inv_rms(float ssum, float kinv, float eps) {
  return __builtin_amdgcn_rsqf(ssum * kinv + eps);
}

// rs[m] = 1 / sqrt(mean_k x[m, k]^2 + eps) from per-thread partial sums of
// squares: shuffles within each wave, then one LDS pass.  Ends with a barrier.
template <int MT, int BLOCK>
__device__ __forceinline__ void rms_finish(float (&part)[MT], int K, float eps, float* rs,
                                           float* scratch /* [BLOCK / 64][MT] */, int tid) {
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) part[m] += __shfl_xor(part[m], o);
  }
  if ((tid & 63) == 0) {
#pragma unroll
    for (int m = 0; m < MT; ++m) scratch[(tid >> 6) * MT + m] = part[m];
  }
  __syncthreads();
  if (tid < MT) {
    float ssum = 0.f;
    for (int w = 0; w < BLOCK / 64; ++w) ssum += scratch[w * MT + tid];
    rs[tid] = inv_rms(ssum, 1.f / float(K), eps);
  }
  __syncthreads();
}

// rs[m] for m < M, any alignment: every thread sums x[m, k]^2 over k = tid,
// tid + BLOCK, ...  Ends with a barrier.
template <typename XT, int MT, int BLOCK>
__device__ __forceinline__ void rms_scales(const XT* __restrict__ x, int M, int K, float eps, float* rs,
                                           float* scratch /* [BLOCK / 64][MT] */, int tid) {
  float part[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) part[m] = 0.f;
  for (int k = tid; k < K; k += BLOCK) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float v = m < M ? to_f32(x[size_t(m) * K + k]) : 0.f;
      part[m] += v * v;
    }
  }
  rms_finish<MT, BLOCK>(part, K, eps, rs, scratch, tid);
}

// 8 effective inputs (m, kb .. kb+7) times g, zeros past K.
template <typename XT>
__device__ __forceinline__ void load_input8(const MfmaParams& p, const float* __restrict__ g, int m, int kb,
                                            float rsm, float (&a)[8]) {
  const XT* __restrict__ x = static_cast<const XT*>(p.x) + size_t(m) * p.K;
  const int K = p.K;
  if (p.xvec && kb + 8 <= K) {
    float gv[8];
    load8(x + kb, a);
    load8(g + kb, gv);
    if (p.xmode == LBK_INPUT_RMSNORM) {
      float wv[8];
      load8(p.nw + kb, wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) gv[i] *= wv[i] * rsm;
    } else if (p.xmode == LBK_INPUT_SILU_MUL) {
      float uv[8];
      load8(static_cast<const XT*>(p.x1) + size_t(m) * K + kb, uv);
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = silu_f(a[i]) * uv[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] *= gv[i];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = 0.f;
      if (kb + i < K) {
        v = to_f32(x[kb + i]) * g[kb + i];
        if (p.xmode == LBK_INPUT_RMSNORM) v *= p.nw[kb + i] * rsm;
        else if (p.xmode == LBK_INPUT_SILU_MUL)
          v = silu_f(to_f32(x[kb + i])) * to_f32(static_cast<const XT*>(p.x1)[size_t(m) * K + kb + i]) * g[kb + i];
      }
      a[i] = v;
    }
  }
}

// Blocks are dispatched to the 8 XCDs of MI355X round-robin: blocks b and
// b + 8 run on the same XCD (measured with HW_REG_XCC_ID; which XCD block 0
// lands on varies between launches).  This maps block b to a logical index
// so that each XCD gets one contiguous range of logical blocks: neighbouring
// k-chunks of a row-block, which share 128-byte lines of the sign rows, then
// meet in one L2 instead of fetching the line from HBM once per XCD.  Any
// other dispatch order only changes the traffic, not the result.
__device__ __forceinline__ int xcd_contiguous_block(int b, int G) {
  const int x = b & 7, j = b >> 3;
  const int q = G >> 3, r = G & 7;  // XCD x holds q + (x < r) blocks
  return x * q + min(x, r) + j;
}

// Fill a compact operand: one thread per chunk; load_row(c, m, a) gives the
// 8 values of chunk c for m < M.  All loads of a block are issued before any
// is used; rows m >= M are written as zeros (their loads read row M - 1).
template <int MT, int BLOCK, typename F>
__device__ __forceinline__ void build_compact(u32x4* lds, int nch, int M, int tid, F&& load_row) {
  using L = Compact<MT>;
  for (int c = tid; c < nch; c += BLOCK) {
#pragma unroll
    for (int mb = 0; mb < L::MB; ++mb) {
      float a[L::MR][8];
#pragma unroll
      for (int ml = 0; ml < L::MR; ++ml) load_row(c, min(mb * 8 + ml, M - 1), a[ml]);
      u32x4* base = lds + (size_t(mb) * nch + c) * L::ROWS;
#pragma unroll
      for (int ml = 0; ml < L::MR; ++ml) {
        u32x4 hi = {0u, 0u, 0u, 0u}, lo = {0u, 0u, 0u, 0u};
        if (mb * 8 + ml < M) split8(a[ml], hi, lo);
        base[ml] = hi;
        base[L::MR + ml] = lo;
      }
      base[2 * L::MR] = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

// RPT rows m0 .. m0 + RPT - 1 of the effective input times g for one chunk of
// 8 k from kb, vector path (x, x1, g and the RMSNorm weight 16-byte aligned,
// K % 8 == 0: a chunk lies wholly inside K or wholly past it).  load() issues
// every load at clamped addresses (rows past M read row M - 1).  get() gives
// row i times g, zero past K -- for RMSNorm x * w * g without the row's 1/rms,
// which multiplies t instead (the expand kernel applies it); sq() gives the
// row's sum of x^2 over the chunk.
template <typename XT, int RPT, int MODE>
struct RowChunk {
  static constexpr bool kSilu = MODE == LBK_INPUT_SILU_MUL;
  Raw8<XT> xr[RPT];
  Raw8<XT> ur[kSilu ? RPT : 1];
  Raw8<float> gr, wr;
  bool valid;

  // rows m0 + i of the block's rows [rb, rb + Mc)
  __device__ __forceinline__ void load(const MfmaParams& p, const float* __restrict__ g, int kb, int m0, int rb,
                                       int Mc) {
    valid = kb < p.K;
    const int kl = valid ? kb : 0;
    const XT* __restrict__ x = static_cast<const XT*>(p.x);
    gr.load(g + kl);
    if constexpr (MODE == LBK_INPUT_RMSNORM) wr.load(p.nw + kl);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const size_t at = size_t(rb + min(m0 + i, Mc - 1)) * p.K + kl;
      xr[i].load(x + at);
      if constexpr (kSilu) ur[i].load(static_cast<const XT*>(p.x1) + at);
    }
  }

  __device__ __forceinline__ void get(int i, float (&a)[8]) const {
    float gv[8];
    gr.get(gv);
    xr[i].get(a);
    if constexpr (MODE == LBK_INPUT_RMSNORM) {
      float wv[8];
      wr.get(wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) gv[e] *= wv[e];
    } else if constexpr (kSilu) {
      float uv[8];
      ur[i].get(uv);
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = silu_f(a[e]) * uv[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = valid ? a[e] * gv[e] : 0.f;
  }

  __device__ __forceinline__ float sq(int i) const {
    float a[8];
    xr[i].get(a);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += a[e] * a[e];
    return valid ? s : 0.f;
  }
};

// The latent kernel's compact A operand of one k-chunk (NCH chunks of 8 k
// from k0), vector path.  The NCH * MT (chunk, row) pairs are spread over the
// block: thread tid takes chunk tid % NCH and RPT rows from RPT * (tid / NCH),
// so consecutive threads read consecutive chunks of a row and no thread holds
// more than RPT rows; waves with no pair skip as a whole.  With ssq (RMSNorm,
// one row-block per k-chunk) the chunk's sums of x^2 of every row m < M are
// added into ssq_out[m].  Ends with this thread's LDS writes, no barrier.
template <typename XT, int MT, int NCH, int MODE>
__device__ __forceinline__ void stage_latent_rows(const MfmaParams& p, const float* __restrict__ g, int k0,
                                                  u32x4* lds, int tid, bool ssq, float* ssq_out, int rb, int Mc) {
  using L = Compact<MT>;
  constexpr int RG = MT < kBlock / NCH ? MT : kBlock / NCH;  // row groups (threads per chunk)
  constexpr int RPT = MT / RG;                                // rows per thread
  constexpr int PAIRS = NCH * RG;                             // active threads
  static_assert(RG * RPT == MT && PAIRS <= kBlock, "row groups");
  if (tid - (tid & 63) >= PAIRS) return;  // the whole wave is idle
  const bool active = tid < PAIRS;
  const int c = tid % NCH;
  const int rg = active ? tid / NCH : 0;
  const int m0 = rg * RPT;
  RowChunk<XT, RPT, MODE> in;
  in.load(p, g, k0 + 8 * c, m0, rb, Mc);
  if constexpr (MODE == LBK_INPUT_RMSNORM) {
    if (ssq) {
      // lanes of one row group are contiguous: reduce over them, then one
      // atomic per row from the group's first lane
      constexpr int SPAN = NCH < 64 ? NCH : 64;
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        float v = active ? in.sq(i) : 0.f;
#pragma unroll
        for (int o = SPAN / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o);
        if (active && (tid % SPAN) == 0 && m0 + i < Mc) {
          if (p.part) {
            // ssq_out is this k-chunk's two sub-slots; a row group of NCH
            // threads spans NCH / SPAN (1 or 2) waves
            // (agent-scope stores: another block of the row-block reads them)
            const int sub = (tid / SPAN) % (NCH / SPAN);
            __hip_atomic_store(ssq_out + sub * kMaxMfmaM + m0 + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (NCH / SPAN == 1)
              __hip_atomic_store(ssq_out + kMaxMfmaM + m0 + i, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          } else {
            unsafeAtomicAdd(ssq_out + m0 + i, v);
          }
        }
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int m = m0 + i;
    const int mb = m / 8, ml = m % 8;
    u32x4* base = lds + (size_t(mb) * NCH + c) * L::ROWS;
    u32x4 hi = {0u, 0u, 0u, 0u}, lo = {0u, 0u, 0u, 0u};
    if (m < Mc) {
      float a[8];
      in.get(i, a);
      split8(a, hi, lo);
    }
    base[ml] = hi;
    base[L::MR + ml] = lo;
  }
  if (rg == 0) {
#pragma unroll
    for (int mb = 0; mb < L::MB; ++mb) lds[(size_t(mb) * NCH + c) * L::ROWS + 2 * L::MR] = u32x4{0u, 0u, 0u, 0u};
  }
}

// LBK_INPUT_ATTN_MERGE, one row: the block's KC = 8 * NCH columns of the
// attention output, merged from the decode attention's per-chunk partials
// (o[hd], m, l of the positions of chunk j; chunks j <= pos / kAttnChunk):
//   x[k] = sum_j exp(m_j - M) o_j[k % hd] / sum_j exp(m_j - M) l_j,  M = max_j m_j
// for head k / hd (the merge of attn_combine_kernel, done by the consumer so
// that the draft step has no merge launch).  Wave w takes chunks w, w + 4, ..
// in rounds of JB whose loads issue together, lane DPL consecutive columns
// (one head); the waves' (max, num, den) are merged through LDS.  A position
// outside [0, max_seq) gives x = 0 (the attention yields zeros there).
template <int NCH>
__device__ __forceinline__ void stage_latent_attn(const MfmaParams& p, const float* __restrict__ g, int k0,
                                                  u32x4* lds, int tid) {
  constexpr int KC = 8 * NCH, DPL = KC / 64, JB = DPL <= 4 ? 12 : DPL == 8 ? 8 : 4;
  static_assert(DPL == 2 || DPL == 4 || DPL == 8 || DPL == 16, "columns per lane");
  __shared__ float w_m[4][64], w_d[4][64];
  __shared__ float w_n[4][KC];
  __shared__ float xs[KC];
  const int wave = tid >> 6, lane = tid & 63;
  // this thread's g chunk (threads c < NCH), loaded before anything waits
  Raw8<float> gr;
  const bool gvalid = tid < NCH && k0 + 8 * tid < p.K;
  if (gvalid) gr.load(g + k0 + 8 * tid);
  const int64_t pos = p.apos ? *p.apos : p.apos_host;
  const int used = (pos >= 0 && pos < p.amax_seq) ? int(pos / kAttnChunk) + 1 : 0;
  const int hd = p.ahd, stride = hd + kAttnPad;
  const int kcol = k0 + lane * DPL;
  const bool cvalid = kcol < p.K;  // DPL divides hd: a lane's columns are wholly inside K or past it
  const int head = cvalid ? kcol / hd : 0;
  const int d = kcol - head * hd;
  const float* __restrict__ ph = static_cast<const float*>(p.x) + size_t(head) * p.achunks * stride;
  float M = -INFINITY, den = 0.f, num[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) num[i] = 0.f;
  for (int j0 = wave; j0 < used; j0 += 4 * JB) {
    float2 ml[JB];
    float ov[JB][DPL];
#pragma unroll
    for (int b = 0; b < JB; ++b) {
      const float* row = ph + size_t(min(j0 + 4 * b, used - 1)) * stride;
      ml[b] = *reinterpret_cast<const float2*>(row + hd);
      if constexpr (DPL == 2) {
        const float2 v = *reinterpret_cast<const float2*>(row + d);
        ov[b][0] = v.x;
        ov[b][1] = v.y;
      } else {
#pragma unroll
        for (int q = 0; q < DPL / 4; ++q) {
          const float4 v = *reinterpret_cast<const float4*>(row + d + 4 * q);
          ov[b][4 * q] = v.x;
          ov[b][4 * q + 1] = v.y;
          ov[b][4 * q + 2] = v.z;
          ov[b][4 * q + 3] = v.w;
        }
      }
    }
    float bm = M;
#pragma unroll
    for (int b = 0; b < JB; ++b)
      if (j0 + 4 * b < used) bm = fmaxf(bm, ml[b].x);
    const float cs = M == -INFINITY ? 0.f : __expf(M - bm);  // bm is finite: chunk j0 < used
    den *= cs;
#pragma unroll
    for (int i = 0; i < DPL; ++i) num[i] *= cs;
#pragma unroll
    for (int b = 0; b < JB; ++b) {
      const float w = j0 + 4 * b < used ? __expf(ml[b].x - bm) : 0.f;
      den += w * ml[b].y;
#pragma unroll
      for (int i = 0; i < DPL; ++i) num[i] += w * ov[b][i];
    }
    M = bm;
  }
  w_m[wave][lane] = M;
  w_d[wave][lane] = den;
#pragma unroll
  for (int i = 0; i < DPL; ++i) w_n[wave][lane * DPL + i] = num[i];
  __syncthreads();
  for (int k = tid; k < KC; k += kBlock) {
    const int ln = k / DPL;
    float mx = fmaxf(fmaxf(w_m[0][ln], w_m[1][ln]), fmaxf(w_m[2][ln], w_m[3][ln]));
    float nn = 0.f, dd = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float e = w_m[w][ln] == -INFINITY ? 0.f : __expf(w_m[w][ln] - mx);
      nn += e * w_n[w][k];
      dd += e * w_d[w][ln];
    }
    xs[k] = (mx == -INFINITY || k0 + k >= p.K) ? 0.f : nn / dd;
  }
  __syncthreads();
  if (tid < NCH) {
    u32x4 hi = {0u, 0u, 0u, 0u}, lo = {0u, 0u, 0u, 0u};
    if (gvalid) {
      float a[8], gv[8];
      gr.get(gv);
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = xs[8 * tid + e] * gv[e];
      split8(a, hi, lo);
    }
    u32x4* base = lds + size_t(tid) * Compact<1>::ROWS;
    base[0] = hi;
    base[Compact<1>::MR] = lo;
    base[2 * Compact<1>::MR] = u32x4{0u, 0u, 0u, 0u};
  }
}

// ---------------------------------------------------------------------------
// Stage 1 (MFMA): t += l * (V_sign . (g*x)) over this block's k-chunk
// grid.x = (row-blocks of all segments) * nkc, block = 256 threads (4 waves)
// LDS: compact A operand of g*x for the k-chunk (KC/8 chunks)
//
// The k-chunks of a row-block add into t with fp32 atomics (t is zero on
// entry); kernel completion publishes t to expand_mfma_kernel.  Atomics
// cost nothing measurable here, unlike an agent-scope fence, which writes
// back the whole L2 of the XCD.  The order of the additions is not fixed,
// so the last bits of t can differ from run to run.  DET (deterministic
// mode, p.part set) is an instantiation of its own: its fixed-order sum
// keeps many loads in flight, and the registers for them would otherwise
// hold every call's kernel to two waves per SIMD.
// ---------------------------------------------------------------------------
template <typename XT, int MT, int WPL, bool DET>
__global__ __launch_bounds__(kBlock) void latent_mfma_kernel(MfmaParams p) {
  using L = Compact<MT>;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  u32x4* lds_a = reinterpret_cast<u32x4*>(lds_raw);
  constexpr int KC = 128 * WPL;
  constexpr int NCH = KC / 8;  // 8-column chunks per k-chunk

  // Logical block lb: each XCD runs a contiguous range of them.  Row-block
  // major (the k-chunks of a row-block on one XCD) when V is read as stored:
  // neighbouring k-chunks then share 128-byte lines of the sign rows.  With
  // V's tiled copy no line spans two k-chunks, and k-chunk major order has
  // each XCD fetch its own share of the input rows instead of all of them.
  const int lb = xcd_contiguous_block(int(blockIdx.x), int(gridDim.x));
  const int nrbt = int(gridDim.x) / p.nkc;  // row-blocks of all segments
  const int kc = p.kc_major ? lb / nrbt : lb % p.nkc;
  const int rbk = p.kc_major ? lb - kc * nrbt : lb / p.nkc;
  // segment of this row-block: a wave-uniform index, so the descriptor is
  // read with scalar loads from the kernel arguments
  int si = 0;
#pragma unroll
  for (int i = 1; i < kMaxSeg; ++i) si += (i < p.nseg && rbk >= p.seg[i].rb0) ? 1 : 0;
  si = __builtin_amdgcn_readfirstlane(si);
  const LatSeg& SG = p.seg[si];
  const int rb = rbk - SG.rb0;
  const int R = SG.R;
  const int RP = SG.RP;
  const int tbase = SG.tbase;
  const float* __restrict__ g = SG.g;
  const float* __restrict__ lvec = SG.l;
  const uint32_t* __restrict__ V = SG.V;
  const int k0 = kc * KC;
  // rows [mrow0, mrow0 + Mc) of the call: the block's row chunk (grid.y);
  // a one-row kernel never runs in chunks, and folding that in at compile
  // time shortens every draft-step call (draft step 1.194 -> 1.174 ms)
  const int mrow0 = MT == 1 ? 0 : int(blockIdx.y) * p.crows;
  const int Mc = MT == 1 ? 1 : min(p.crows, p.M - mrow0);
  const int tb = tbase + mrow0 * RP;  // t of the chunk's first row in this segment
  const int tid = int(threadIdx.x);
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int col = lane & 15;   // MFMA column = latent row within the tile
  const int grp = lane >> 4;   // k group 0..3
  const int r = rb * kRowBlock + wave * 16 + col;
  const int w0 = kc * (KC / 32) + grp * WPL;

  // Sign words first, so that their latency overlaps the A-operand build.
  // Every load is issued on every path (clamped addresses: rows past R are
  // never stored, and words past the row meet A columns past K, which are
  // zero), so that no wait has to cover a path that skipped a load.
  uint32_t words[WPL];
  if (SG.Vt) {
    // tiled copy [ceil(R/16)][ceil(KW/4)][16 rows][4 words]: the lane's WPL
    // words are WPL/4 whole 16-byte cells of its row (half a cell at WPL = 2),
    // and the lanes of a load read whole 128-byte lines.  Rows past R read
    // row 0 (never stored); cells past the row read cell 0 (they meet A
    // columns past K, which are zero), as in the untiled path.
    const int kw4 = (p.KW + 3) >> 2;
    const int rr = r < R ? r : 0;
    const uint32_t* __restrict__ cells = SG.Vt + size_t(rr >> 4) * kw4 * 64 + (rr & 15) * 4;
    if constexpr (WPL == 2) {
      const int gi = w0 < p.KW ? w0 >> 2 : 0;
      const uint2 v = *reinterpret_cast<const uint2*>(cells + size_t(gi) * 64 + (w0 & 3));
      words[0] = v.x;
      words[1] = v.y;
    } else {
#pragma unroll
      for (int q = 0; q < WPL / 4; ++q) {
        const int gi = (w0 >> 2) + q < kw4 ? (w0 >> 2) + q : 0;
        const uint4 v = *reinterpret_cast<const uint4*>(cells + size_t(gi) * 64);
        words[4 * q] = v.x;
        words[4 * q + 1] = v.y;
        words[4 * q + 2] = v.z;
        words[4 * q + 3] = v.w;
      }
    }
  } else {
    const uint32_t* __restrict__ vrow = V + size_t(r < R ? r : 0) * p.KW;
    if (p.wvec) {
      // the lane's WPL words in one or two vector loads: with KW % WPL == 0 a
      // lane's words lie wholly inside the row or wholly past it
      const uint32_t* __restrict__ src = vrow + (w0 < p.KW ? w0 : 0);
      if constexpr (WPL == 2) {
        const uint2 v = *reinterpret_cast<const uint2*>(src);
        words[0] = v.x;
        words[1] = v.y;
      } else {
#pragma unroll
        for (int q = 0; q < WPL / 4; ++q) {
          const uint4 v = *reinterpret_cast<const uint4*>(src + 4 * q);
          words[4 * q] = v.x;
          words[4 * q + 1] = v.y;
          words[4 * q + 2] = v.z;
          words[4 * q + 3] = v.w;
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < WPL; ++s) words[s] = vrow[min(w0 + s, p.KW - 1)];
    }
  }
  const float lv = lvec[min(r, R - 1)];
  const float lr = r < R ? lv : 0.f;
  // Latent-buffer state.  Plain loads: within this launch only block 0
  // writes sync[1] and sync[2 + h], which no block of it reads.
  const uint32_t h = p.sync[0] & 1u;
  const uint32_t s0 = p.sync[2];
  const uint32_t s1 = p.sync[3];

  // ---- A operand: hi/lo bf16 of g[k] * input[m, k] for this k-chunk ----
  if (p.xvec) {
    // RMSNorm: t is accumulated without the rows' 1/rms; the blocks of the
    // first row-block add their chunk's sums of squares next to t, and the
    // expand kernel scales t by 1/rms when it stages it
    float* ssq_out = p.part   ? p.part + size_t(p.nkc) * p.tsize + size_t(2 * kc) * kMaxMfmaM
                     : p.tdst ? p.tdst + p.tsize + mrow0
                              : p.t2 + size_t(h) * kTHalf + p.tsize + mrow0;
    if (MT == 1 && p.xmode == LBK_INPUT_ATTN_MERGE) {
      if constexpr (MT == 1) stage_latent_attn<NCH>(p, g, k0, lds_a, tid);
    } else if (p.xmode == LBK_INPUT_RMSNORM)
      stage_latent_rows<XT, MT, NCH, LBK_INPUT_RMSNORM>(p, g, k0, lds_a, tid, rbk == 0, ssq_out, mrow0, Mc);
    else if (p.xmode == LBK_INPUT_SILU_MUL)
      stage_latent_rows<XT, MT, NCH, LBK_INPUT_SILU_MUL>(p, g, k0, lds_a, tid, false, ssq_out, mrow0, Mc);
    else
      stage_latent_rows<XT, MT, NCH, LBK_INPUT_PLAIN>(p, g, k0, lds_a, tid, false, ssq_out, mrow0, Mc);
  } else {
    __shared__ float rs[MT];
    if (p.xmode == LBK_INPUT_RMSNORM) {
      __shared__ float rscratch[kBlock / 64 * MT];
      rms_scales<XT, MT, kBlock>(static_cast<const XT*>(p.x) + size_t(mrow0) * p.K, Mc, p.K, p.eps, rs, rscratch,
                                 tid);
    }
    build_compact<MT, kBlock>(lds_a, NCH, Mc, tid, [&](int c, int m, float (&a)[8]) {
      load_input8<XT>(p, g, mrow0 + m, k0 + 8 * c, p.xmode == LBK_INPUT_RMSNORM ? rs[m] : 1.f, a);
    });
  }
  __syncthreads();

  uint32_t kmask = 0x80008000u, kone = 0x3F803F80u;
  asm volatile("" : "+v"(kmask), "+v"(kone));
  const int lrow = L::lane_row(col);
  f32x4 acc[L::MB];
#pragma unroll
  for (int i = 0; i < L::MB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < WPL; ++s) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x8 bop = signs_to_bf16x8(words[s], j, kmask, kone);
      const int c = (grp * WPL + s) * 4 + j;
#pragma unroll
      for (int mb = 0; mb < L::MB; ++mb) {
        const bf16x8 aop = __builtin_bit_cast(bf16x8, lds_a[(size_t(mb) * NCH + c) * L::ROWS + lrow]);
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop, acc[mb], 0, 0, 0);
      }
    }
  }

  // C rows 4*grp + i: grp 0,1 = hi of m = 4*grp + i, grp 2,3 = lo of the same m.
  float sum[L::MB][4];
#pragma unroll
  for (int mb = 0; mb < L::MB; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) sum[mb][i] = add_upper32(acc[mb][i]);

  float* trow = (p.tdst ? p.tdst : p.t2 + size_t(h) * kTHalf) + tb + r;
  if constexpr (DET) {
    // Deterministic mode: this k-chunk's partials go to part[kc] through
    // agent-scope stores (the row-block's blocks run on any XCD); once they
    // have landed the block counts itself in, and the row-block's last block
    // adds all nkc partials of its rows in chunk order, so the sum does not
    // depend on which block finished when.
    float* __restrict__ mine = p.part + size_t(tb) + r;
    if (lane < 32 && r < R) {
#pragma unroll
      for (int mb = 0; mb < L::MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = mb * 8 + grp * 4 + i;
          if (m < Mc)
            __hip_atomic_store(mine + size_t(kc) * p.tsize + size_t(m) * RP, lr * sum[mb][i], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    __shared__ int s_last;
    __syncthreads();
    if (tid == 0) {
      const uint32_t before = __hip_atomic_fetch_add(p.det_cnt + rbk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = before + 1u == uint32_t(p.nkc) ? 1 : 0;
    }
    __syncthreads();
    if (s_last) {
      // Each output (m, row) is the sum of nkc partials in chunk order,
      // split into four contiguous quarters of the chunks, one per wave:
      // each wave issues its quarter's loads for G rows of M at once (they
      // are independent; summed in order afterwards), then wave 0 adds the
      // four quarter sums in order.  The grouping is fixed, so the result
      // is too.  The A-operand LDS is free by now and holds the quarter sums.
      constexpr int G = MT < 4 ? MT : 4;
      static_assert(size_t(L::MB) * NCH * L::ROWS * 16 >= (4 * G * kRowBlock + 4 * kMaxMfmaM) * sizeof(float),
                    "quarter sums fit in the A-operand LDS");
      float* red = reinterpret_cast<float*>(lds_a);  // [quarter][G][kRowBlock]
      float* rss = red + 4 * G * kRowBlock;           // [quarter][kMaxMfmaM]
      const int rl = tid % kRowBlock;
      const int qt = tid / kRowBlock;
      const int rr = rb * kRowBlock + rl;
      const int c0 = p.nkc * qt / 4, c1 = p.nkc * (qt + 1) / 4;
      constexpr int B = 8;  // loads in flight per row of M
      if (p.late_rs && rbk == 0) {
        // an RMSNorm input's sums of squares: the first row-block's
        // k-chunks wrote them (sub-slots 2 kc and 2 kc + 1)
        float a = 0.f;
        if (rl < Mc) {
          const float* __restrict__ ssq = p.part + size_t(p.nkc) * p.tsize + rl;
          for (int j = 2 * c0; j < 2 * c1; j += B) {
            float v[B];
#pragma unroll
            for (int u = 0; u < B; ++u)
              v[u] = j + u < 2 * c1 ? __hip_atomic_load(ssq + size_t(j + u) * kMaxMfmaM, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT)
                                    : 0.f;
#pragma unroll
            for (int u = 0; u < B; ++u)
              if (j + u < 2 * c1) a += v[u];
          }
        }
        if (rl < kMaxMfmaM) rss[qt * kMaxMfmaM + rl] = a;
      }
      float* __restrict__ tout = p.t2 + size_t(h) * kTHalf + tb + rr;
      const float* __restrict__ src = p.part + size_t(tb) + rr;
      for (int mg = 0; mg < Mc; mg += G) {
        float a[G];
#pragma unroll
        for (int i = 0; i < G; ++i) a[i] = 0.f;
        if (rr < R) {
          for (int c = c0; c < c1; c += B) {
            float v[G][B];
#pragma unroll
            for (int i = 0; i < G; ++i)
#pragma unroll
              for (int u = 0; u < B; ++u)
                v[i][u] = mg + i < Mc && c + u < c1
                              ? __hip_atomic_load(src + size_t(c + u) * p.tsize + size_t(mg + i) * RP,
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                              : 0.f;
#pragma unroll
            for (int i = 0; i < G; ++i)
#pragma unroll
              for (int u = 0; u < B; ++u)
                if (c + u < c1) a[i] += v[i][u];
          }
        }
#pragma unroll
        for (int i = 0; i < G; ++i) red[(qt * G + i) * kRowBlock + rl] = a[i];
        __syncthreads();
        if (qt == 0 && rr < R) {
#pragma unroll
          for (int i = 0; i < G; ++i) {
            const int m = mg + i;
            if (m < Mc) {
              float s = red[i * kRowBlock + rl];
#pragma unroll
              for (int q = 1; q < 4; ++q) s += red[(q * G + i) * kRowBlock + rl];
              tout[size_t(m) * RP] = s;
            }
          }
        }
        if (mg == 0 && p.late_rs && rbk == 0 && tid < Mc) {
          float s = rss[tid];
#pragma unroll
          for (int q = 1; q < 4; ++q) s += rss[q * kMaxMfmaM + tid];
          p.t2[size_t(h) * kTHalf + p.tsize + mrow0 + tid] = s;
        }
        __syncthreads();
      }
      if (tid == 0) __hip_atomic_store(p.det_cnt + rbk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
    if (lane < 32 && r < R) {
#pragma unroll
      for (int mb = 0; mb < L::MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = mb * 8 + grp * 4 + i;
          if (m < Mc) {
            if (p.nkc == 1) trow[size_t(m) * RP] = lr * sum[mb][i];
            else unsafeAtomicAdd(trow + size_t(m) * RP, lr * sum[mb][i]);
          }
        }
    }
  }

  // clear this block's slice of the other half; publish the state
  const int nblk = int(gridDim.x * gridDim.y);
  const int bl = int(blockIdx.x + blockIdx.y * gridDim.x);
  if (p.tdst) {
    // a chain's first call: its own region, and the region given to clear
    const int per = (p.nclr + nblk - 1) / nblk;
    const int hi = min(p.nclr, (bl + 1) * per);
    for (int i = bl * per + tid; i < hi; i += kBlock) p.clr[i] = 0.f;
  } else {
    const uint32_t stale = h ? s0 : s1;
    float* __restrict__ other = p.t2 + size_t(h ^ 1u) * kTHalf;
    const int per = int((stale + unsigned(nblk) - 1) / unsigned(nblk));
    const int lo = bl * per;
    const int hi = min(int(stale), lo + per);
    for (int i = lo + tid; i < hi; i += kBlock) other[i] = 0.f;
    if (bl == 0 && tid == 0) {
      __hip_atomic_store(p.sync + 1, h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.sync + 2 + h, uint32_t(p.tsize + kSsqSlots), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // rank-sliced expand: y starts as bias + residual (the residual may be y
  // itself), and the slices add their parts to it
  if (MT > 1 && p.ks > 1) {
    for (int q = 0; q < p.nproj; ++q) {
      const ExpProj& P = p.proj[q];
      float* y = static_cast<float*>(P.y);  // not restrict: P.res may be y
      const int64_t total = int64_t(p.M) * P.N;
      for (int64_t i = int64_t(bl) * kBlock + tid; i < total; i += int64_t(nblk) * kBlock) {
        const float b = P.bias ? P.bias[i % P.N] : 0.f;
        y[i] = P.res ? P.res[i] + b : b;
      }
    }
  }
}

// A projection's branches as the expand kernel's waves walk them: the rank
// steps (4 sign words of a U row) of branch 0, padded to a multiple of 4
// when branch 1 follows (P0 steps), then those of branch 1, so that no group
// of 4 consecutive steps from a multiple of 4 spans both branches.  With one
// branch, "branch 1" repeats branch 0 from P0 = its step count (no group
// reaches it).  Fields are wave-uniform.
struct StepSeq {
  const uint32_t* U[2];
  int RW[2];     // words per U row
  int steps[2];  // RWp / 4
  int P0;
  int N;
};

// Sign words of a wave's steps [q0, q1) of a StepSeq, q0 a multiple of 4.
// Full groups take one 16-byte load per lane: lane grp g takes the 4 words of
// step q0 + 4t + g and uses word u in MFMA iteration u of group t, so the 4
// lanes of a row read 64 contiguous bytes.  The (q1 - q0) % 4 steps left at
// the end of the sequence take one word per lane, word 4 * step + g.  Every
// lane issues S / 4 + 3 loads whatever the range is (clamped addresses), so
// that waits on earlier loads stay exact.  A 16-byte load may run past its row
// into the next one (those words meet ranks past R, whose t is zero); at the
// end of the matrix (N * RW >= 4 words) the load start is clamped and sh
// records by how many words the lane's words sit further on.
template <int S>
struct SignWords {
  uint32_t grp[S / 4][4];
  int sh[S / 4];
  uint32_t rem[3];

  __device__ __forceinline__ void load(const StepSeq& b, int row, int q0, int q1, int g) {
    const int G = (q1 - q0) >> 2;
#pragma unroll
    for (int t = 0; t < S / 4; ++t) {
      const bool b1 = q0 + 4 * t >= b.P0;  // the group's branch (uniform)
      const uint32_t* __restrict__ U = b1 ? b.U[1] : b.U[0];
      const int RW = b1 ? b.RW[1] : b.RW[0];
      const int nst = b1 ? b.steps[1] : b.steps[0];
      const int st = min((b1 ? q0 + 4 * t - b.P0 : q0 + 4 * t) + g, nst - 1);
      const int64_t gi = int64_t(row) * RW + 4 * st;
      const int64_t last = int64_t(b.N) * RW - 4;
      const int64_t gl = gi < last ? gi : last;
      uint4 v;
      __builtin_memcpy(&v, U + gl, 16);
      grp[t][0] = v.x;
      grp[t][1] = v.y;
      grp[t][2] = v.z;
      grp[t][3] = v.w;
      sh[t] = int(gi - gl);
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int q = q0 + 4 * G + i;
      const bool b1 = q >= b.P0;
      const uint32_t* __restrict__ U = b1 ? b.U[1] : b.U[0];
      const int RW = b1 ? b.RW[1] : b.RW[0];
      const int st = min(b1 ? q - b.P0 : q, (b1 ? b.steps[1] : b.steps[0]) - 1);
      rem[i] = U[int64_t(row) * RW + min(4 * st + g, RW - 1)];
    }
  }

  // the 4 words of group t in step order (after an end-of-matrix shift)
  __device__ __forceinline__ void group(int t, uint32_t (&w)[4]) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = grp[t][e];
    if (__builtin_amdgcn_ballot_w64(sh[t] != 0)) {
      const int k = sh[t];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t a1 = grp[t][min(e + 1, 3)], a2 = grp[t][min(e + 2, 3)], a3 = grp[t][3];
        w[e] = k == 0 ? w[e] : k == 1 ? a1 : k == 2 ? a2 : a3;
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Stage 2 (MFMA): y = bias + sum_b h_b * (U_b_sign . t_b) [+ residual] per
// projection.  block = WAVES waves over 16 * tiles output rows of one
// projection, tiles = WAVES / splits, and rank slice blockIdx.y of ks: the
// projection's StepSeq cut into ks slices of a multiple of 4 steps.  Wave w
// owns row tile w % tiles and part w / tiles of the block's slice (with two
// branches a multiple of 4 steps per part); the splits parts of a tile meet
// in LDS.  A block stages the t chunks of its slice only.  With ks = 1 it
// writes y; with ks > 1 the latent kernel has set y = bias + residual and each
// slice adds its part with fp32 atomics.  The host picks WAVES, splits, ks.
// grid = (sum over projections of ceil(N / (16 * tiles)), ks)
// LDS: compact A operands of the slice's t chunks, branch 0's then branch 1's
//
// Loads are issued in the order they are needed -- the latent-buffer half
// (the staging addresses depend on it), each thread's first staging tasks,
// the sign words group by group, then h, bias and residual -- at clamped
// addresses: rows past N are never stored, and sign words past a row meet
// ranks past R, whose t is zero.  Vector-memory waits retire loads in issue
// order, so the staging waits for its own loads only and the MFMA loop for
// one group of sign words at a time, while the rest are still arriving.
// ---------------------------------------------------------------------------
// 8-wave blocks of the 8-row kernel with up to 24 steps per wave are held to
// 128 VGPRs (four waves per SIMD: two blocks per CU); at 24 steps that
// spills two dwords and let q/k/v's 480 blocks at 33 rows run in one round
// (33.6 -> 32.1 us per call).  At 32 steps it would spill 96 bytes per lane.
template <typename YT, int MT, int S, int WAVES>
__global__ __launch_bounds__(WAVES * kWave, WAVES == 8 && MT == 8 && S <= 24 ? 4 : 1) void expand_mfma_kernel(
    MfmaParams p) {
  using L = Compact<MT>;
  constexpr int THREADS = WAVES * kWave;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  u32x4* lds_t = reinterpret_cast<u32x4*>(lds_raw);
  __shared__ float red[WAVES][L::MB * 4][32];
  const int tid = int(threadIdx.x);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform
  const int lane = tid % kWave;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int splits = p.splits;
  const int tiles = WAVES / splits;
  const int tile = wave % tiles;
  const int part = wave / tiles;
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxProj; ++i) pi += (i < p.nproj && int(blockIdx.x) >= p.proj[i].tile0) ? 1 : 0;
  pi = __builtin_amdgcn_readfirstlane(pi);
  const ExpProj& P = p.proj[pi];
  const int n = (int(blockIdx.x) - P.tile0) * 16 * tiles + tile * 16 + col;
  const bool nvalid = n < P.N;
  const int nc = nvalid ? n : 0;
  // rows [mrow0, mrow0 + M) of the call: the block's row chunk (grid.z)
  const int mrow0 = MT == 1 ? 0 : int(blockIdx.z) * p.crows;
  const int M = MT == 1 ? 1 : min(p.crows, p.M - mrow0);
  const bool two = P.nb > 1;
  // half of the latent buffer the latent kernel of this call filled (only
  // block 0 writes the state here, and only sync[0]).  Read first, with a
  // vector load (the index is opaque to the compiler), so that the wait for it
  // holds none of the loads issued after it
  int zero = 0;
  asm volatile("" : "+v"(zero));
  const uint32_t hq_word = p.sync[1 + zero];
  __builtin_amdgcn_sched_barrier(0);

  // the projection's steps in sequence and this wave's part [q0, q1) of them
  StepSeq sq;
  sq.U[0] = P.U[0];
  sq.U[1] = P.U[two ? 1 : 0];
  sq.RW[0] = __builtin_amdgcn_readfirstlane(P.RW[0]);
  sq.RW[1] = __builtin_amdgcn_readfirstlane(P.RW[two ? 1 : 0]);
  sq.steps[0] = __builtin_amdgcn_readfirstlane(P.RWp[0] / 4);
  sq.steps[1] = __builtin_amdgcn_readfirstlane(P.RWp[two ? 1 : 0] / 4);
  sq.P0 = two ? (sq.steps[0] + 3) & ~3 : sq.steps[0];
  sq.N = P.N;
  const int nsteps = sq.P0 + (two ? sq.steps[1] : 0);
  // the block's slice [sb0, sb1) of the sequence: slice s takes groups of 4
  // steps [s * ng / ks, (s + 1) * ng / ks) (so no group spans P0); a slice of
  // a projection with fewer groups than slices may be empty
  const int ks = MT == 1 ? 1 : p.ks;  // one-row calls are planned without rank slices
  const int ng = (nsteps + 3) / 4;
  const int sb0 = min(4 * (int(blockIdx.y) * ng / ks), nsteps);
  const int sb1 = min(4 * ((int(blockIdx.y) + 1) * ng / ks), nsteps);
  // (a chain's last call does not wait for the word)
  const uint32_t hq = p.tsrc ? 0u : __builtin_amdgcn_readfirstlane(hq_word) & 1u;
  if (p.tsrc) {
    // a chain's last call: t from its region; every block clears its share
    // of the region given to clear
    const int nblk = int(gridDim.x * gridDim.y * gridDim.z);
    const int bl = int(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
    const int per = (p.nclr + nblk - 1) / nblk;
    const int hi = min(p.nclr, (bl + 1) * per);
    for (int i = bl * per + tid; i < hi; i += THREADS) p.clr[i] = 0.f;
  } else if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && tid == 0) {
    // block (0, 0, 0) hands the latent buffer on (P = 1 - Q), before any return
    __hip_atomic_store(p.sync, hq ^ 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (sb0 >= sb1 || int(blockIdx.x) >= p.ntiles) return;
  // parts of a two-branch sequence start at multiples of 4 (no group spans P0)
  const int len = sb1 - sb0;
  const int per = two ? 4 * ((len + 4 * splits - 1) / (4 * splits)) : (len + splits - 1) / splits;
  const int q0 = sb0 + min(part * per, len);
  const int q1 = min(q0 + per, sb1);

  // (1) this thread's first staging tasks (below) go first, the sign words
  // and epilogue operands after them: vector-memory waits retire loads in
  // issue order, so the staging waits for its own loads only, and the MFMA
  // loop waits for each group of sign words as it needs it.  Branch b's
  // chunks [cb, cb + nchb) of its 16 * steps (16 chunks of 8 ranks per
  // step); with ks = 1 all of them
  const int c0a = 16 * min(sb0, sq.steps[0]);
  const int nch0 = 16 * min(sb1, sq.steps[0]) - c0a;
  const int c1a = two ? 16 * min(max(sb0 - sq.P0, 0), sq.steps[1]) : 0;
  const int nch1 = two ? 16 * min(max(sb1 - sq.P0, 0), sq.steps[1]) - c1a : 0;
  const int nch = nch0 + nch1;
  const float* __restrict__ ta = p.tsrc ? p.tsrc : p.t2 + size_t(hq) * kTHalf;
  const float* __restrict__ tssq = ta + p.tsize + mrow0;  // the chunk's rows' sums of squares
  u32x4* tb0 = lds_t;
  u32x4* tb1 = lds_t + size_t(L::MB) * nch0 * L::ROWS;
  // branch fields in scalar registers: a per-lane choice between two fields
  // of the kernel arguments would otherwise become a vector load of the
  // argument block, which every chunk load then waits for
  const int tbase0 = __builtin_amdgcn_readfirstlane(P.tbase[0]);
  const int tbase1 = __builtin_amdgcn_readfirstlane(P.tbase[1]);
  const int rp0 = __builtin_amdgcn_readfirstlane(P.RP[0]);
  const int rp1 = __builtin_amdgcn_readfirstlane(P.RP[1]);
  // The staging in tasks.  Task h holds part h % PARTS of chunk h / PARTS of
  // the slice's chunks of both branches in sequence, every stored row.  With
  // 8 or more rows a task is half a chunk (4 ranks: one 16-byte load per row,
  // so the 64 lanes of a load read 1 KB in one piece rather than every other
  // 16 bytes of 2 KB), and a thread issues two tasks' loads before it waits;
  // with fewer rows a task is a whole chunk.
  constexpr int PARTS = MT >= 8 ? 2 : 1;
  constexpr int W = 8 / PARTS;  // ranks of a task
  constexpr int NV = W / 4;     // 16-byte loads per row
  using Rows = float4[L::MB][L::MR][NV];
  const int ntask = PARTS * nch;
  auto load_task = [&](int h, Rows& v) {
    const int q = h / PARTS;
    const bool b1 = q >= nch0;
    const float* __restrict__ src =
        ta + (b1 ? tbase1 + 8 * (c1a + q - nch0) : tbase0 + 8 * (c0a + q)) + W * (h % PARTS);
    const int rp = b1 ? rp1 : rp0;
#pragma unroll
    for (int mb = 0; mb < L::MB; ++mb)
#pragma unroll
      for (int ml = 0; ml < L::MR; ++ml)
#pragma unroll
        for (int i = 0; i < NV; ++i)
          v[mb][ml][i] = *reinterpret_cast<const float4*>(src + size_t(mrow0 + min(mb * 8 + ml, M - 1)) * rp + 4 * i);
  };
  // 1/rms of each row when t was accumulated without it (RMSNorm input):
  // the rows' sums of squares follow t in the same half, 16-byte aligned (t
  // is a multiple of 128 floats), read with 16-byte loads
  Raw8<float> ssq[(MT + 7) / 8];
  float rsv[MT];  // set before the staging: 1/rms, or 1
  auto put_task = [&](int h, const Rows& v) {
    const int q = h / PARTS;
    const bool b1 = q >= nch0;
    const int c = b1 ? q - nch0 : q;
    u32x4* base0 = b1 ? tb1 : tb0;
    const int nchb = b1 ? nch1 : nch0;
#pragma unroll
    for (int mb = 0; mb < L::MB; ++mb) {
      // the task's W / 2 dwords of each 16-byte row of the chunk
      uint32_t* base = reinterpret_cast<uint32_t*>(base0 + (size_t(mb) * nchb + c) * L::ROWS) + (W / 2) * (h % PARTS);
#pragma unroll
      for (int ml = 0; ml < L::MR; ++ml) {
        uint32_t hi[W / 2], lo[W / 2];
#pragma unroll
        for (int d = 0; d < W / 2; ++d) hi[d] = lo[d] = 0u;
        if (mb * 8 + ml < M) {
          const float r = rsv[mb * 8 + ml];
          float a[W];
#pragma unroll
          for (int i = 0; i < NV; ++i) {
            a[4 * i] = v[mb][ml][i].x * r;
            a[4 * i + 1] = v[mb][ml][i].y * r;
            a[4 * i + 2] = v[mb][ml][i].z * r;
            a[4 * i + 3] = v[mb][ml][i].w * r;
          }
          split_pairs<W>(a, hi, lo);
        }
        store_dwords<W / 2>(base + 4 * ml, hi);
        store_dwords<W / 2>(base + 4 * (L::MR + ml), lo);
      }
      uint32_t z[W / 2];
#pragma unroll
      for (int d = 0; d < W / 2; ++d) z[d] = 0u;
      store_dwords<W / 2>(base + 4 * (2 * L::MR), z);
    }
  };
  Rows v[PARTS];
  // waves with no task skip
  if (tid - lane < ntask) load_task(min(tid, ntask - 1), v[0]);
  if constexpr (PARTS == 2) {
    if (tid - lane + THREADS < ntask) load_task(min(tid + THREADS, ntask - 1), v[1]);
  }
  const bool late = p.late_rs != 0;
  if (late) {
#pragma unroll
    for (int i = 0; i < (MT + 7) / 8; ++i) ssq[i].load(tssq + 8 * i);
  }
  auto put_first = [&]() {
#pragma unroll
    for (int m = 0; m < MT; ++m) rsv[m] = 1.f;
    if (late) {
      const float kinv = 1.f / float(p.K), eps = p.eps;
#pragma unroll
      for (int i = 0; i < (MT + 7) / 8; ++i) {
        float a[8];
        ssq[i].get(a);
#pragma unroll
        for (int e = 0; e < 8 && 8 * i + e < MT; ++e) rsv[8 * i + e] = inv_rms(a[e], kinv, eps);
      }
    }
    if (tid < ntask) put_task(tid, v[0]);
    if constexpr (PARTS == 2) {
      if (tid + THREADS < ntask) put_task(tid + THREADS, v[1]);
    }
  };
  // A slice with more tasks than PARTS * THREADS stages them all here, before
  // the sign words are issued: a loop of loads and waits between the sign
  // loads and the MFMA loop would leave the compiler one full wait for all of
  // them, which the staged order below exists to avoid
  const bool tail = ntask > PARTS * THREADS;  // block-uniform
  if (tail) {
    put_first();
    for (int h = tid + PARTS * THREADS; h < ntask; h += THREADS) {
      load_task(h, v[0]);
      put_task(h, v[0]);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // (2) sign words of the wave's steps
  SignWords<S> sw;
  sw.load(sq, nc, q0, q1, grp);
  // (3) epilogue operands: h, bias, residual rows m = 8 mb + 4 (grp & 1) + i
  const float h0v = P.h[0][nc];
  const float h1v = P.h[two ? 1 : 0][nc];
  const float* __restrict__ bsrc = P.bias ? P.bias : P.h[0];
  const float bnv = bsrc[nc];
  const bool addres = P.res && ks == 1;  // ks > 1: y already holds the residual
  const float* __restrict__ rsrc = addres ? P.res : P.h[0];
  const size_t rstride = addres ? size_t(P.N) : 0;  // no residual: every load reads h[0][0]
  const int rcol = addres ? nc : 0;
  float resv[L::MB][4];
#pragma unroll
  for (int mb = 0; mb < L::MB; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      resv[mb][i] = rsrc[size_t(mrow0 + min(mb * 8 + (grp & 1) * 4 + i, M - 1)) * rstride + rcol];
  __builtin_amdgcn_sched_barrier(0);

  // (4) staging of the first PARTS tasks (when the slice has no more)
  if (!tail) put_first();
  __syncthreads();

  // (5) MFMA over the wave's steps, branch 0 then branch 1: acc holds the
  // branch being walked; on entering branch 1 it moves to acc0
  uint32_t kmask = 0x80008000u, kone = 0x3F803F80u;
  asm volatile("" : "+v"(kmask), "+v"(kone));
  const int lrow = L::lane_row(col);
  f32x4 acc[L::MB], acc0[L::MB];
#pragma unroll
  for (int mb = 0; mb < L::MB; ++mb) {
    acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc0[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  bool in1 = false;  // acc holds branch 1 (wave-uniform)
  auto enter = [&](bool b1) {
    if (b1 && !in1) {
#pragma unroll
      for (int mb = 0; mb < L::MB; ++mb) {
        acc0[mb] = acc[mb];
        acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      in1 = true;
    }
  };
  // 4 MFMAs over word w of the lane's step (chunks 4w .. 4w + 3 of the
  // branch's t); km = ko = 0 gives a zero B operand
  auto mfma4 = [&](uint32_t word, const u32x4* __restrict__ tb, int nchb, int w, uint32_t km, uint32_t ko) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x8 bop = signs_to_bf16x8(word, j, km, ko);
#pragma unroll
      for (int mb = 0; mb < L::MB; ++mb) {
        const bf16x8 aop = __builtin_bit_cast(bf16x8, tb[(size_t(mb) * nchb + 4 * w + j) * L::ROWS + lrow]);
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop, acc[mb], 0, 0, 0);
      }
    }
  };
  {
    const int n = q1 - q0, G = n >> 2, r = n & 3;
#pragma unroll
    for (int t = 0; t < S / 4; ++t) {
      if (t >= G) continue;
      const bool b1 = q0 + 4 * t >= sq.P0;
      enter(b1);
      uint32_t w4[4];
      sw.group(t, w4);
      // this lane's step of the group within its branch, counted from the
      // slice's first step of that branch; steps in branch 0's padding get a
      // zero B operand (and read the slice's first chunks: a slice holding
      // padding holds steps of branch 0 too)
      const int st = (b1 ? q0 + 4 * t - sq.P0 : q0 + 4 * t) + grp;
      const bool valid = b1 || st < sq.steps[0];
      const int sv = valid ? st - (b1 ? c1a : c0a) / 16 : 0;
      const uint32_t km = valid ? kmask : 0u, ko = valid ? kone : 0u;
#pragma unroll
      for (int u = 0; u < 4; ++u) mfma4(w4[u], b1 ? tb1 : tb0, b1 ? nch1 : nch0, 4 * sv + u, km, ko);
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (i >= r) continue;
      const int q = q0 + 4 * G + i;
      const bool b1 = q >= sq.P0;
      enter(b1);
      mfma4(sw.rem[i], b1 ? tb1 : tb0, b1 ? nch1 : nch0, 4 * (b1 ? q - sq.P0 - c1a / 16 : q - c0a / 16) + grp, kmask,
            kone);
    }
  }
  if (!in1) {
#pragma unroll
    for (int mb = 0; mb < L::MB; ++mb) {
      acc0[mb] = acc[mb];
      acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // h-weighted branch sums; C rows 4*grp + i (grp 0,1 hi, 2,3 lo of the same m)
  const float h1 = two ? h1v : 0.f;
  float out[L::MB][4];
#pragma unroll
  for (int mb = 0; mb < L::MB; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      out[mb][i] = h0v * add_upper32(acc0[mb][i]) + h1 * add_upper32(acc[mb][i]);

  // (6) the other parts of the tile add theirs through LDS
  if (splits > 1) {
    if (part > 0 && lane < 32) {
#pragma unroll
      for (int mb = 0; mb < L::MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][mb * 4 + i][lane] = out[mb][i];
    }
    __syncthreads();
    if (part == 0) {
      for (int s = 1; s < splits; ++s) {
#pragma unroll
        for (int mb = 0; mb < L::MB; ++mb)
#pragma unroll
          for (int i = 0; i < 4; ++i) out[mb][i] += red[tile + s * tiles][mb * 4 + i][lane & 31];
      }
    }
  }
  if (part == 0 && lane < 32 && nvalid) {
    YT* y = static_cast<YT*>(P.y);
    const int N = P.N;
    if constexpr (sizeof(YT) == 4) {
      if (ks > 1) {
#pragma unroll
        for (int mb = 0; mb < L::MB; ++mb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = mb * 8 + grp * 4 + i;
            if (m < M) unsafeAtomicAdd(y + size_t(mrow0 + m) * N + n, out[mb][i]);
          }
      }
    }
    if (ks == 1) {
      const float bn = P.bias ? bnv : 0.f;
#pragma unroll
      for (int mb = 0; mb < L::MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = mb * 8 + grp * 4 + i;
          if (m < M) store_out(y, size_t(mrow0 + m) * N + n, out[mb][i] + bn + (P.res ? resv[mb][i] : 0.f));
        }
    }
  }
}

// ---------------------------------------------------------------------------
// Chains (one row, fp32): calls ("links") each of which reads the outputs of
// the link before it -- o, gate/up, down and the next layer's q/k/v of a
// decode step, which the reference runs as one call per layer with thread
// barriers between its stages (patches/littlebit_cpu_optimized.cpp:
// 1627-1833).  The latent stage of link j + 1 sums over its input's k; the
// k-chunk [c0, c0 + C) of that input is rows [c0, c0 + C) of link j's
// outputs.  So one kernel does both: a block expands C = 16 W output rows of
// the NT projections of link j that link j + 1 reads (gate and up for SiLU *
// up, else the one projection) and, with those rows still in registers, adds
// the k-chunk's part of link j + 1's latent vector into its region with fp32
// atomics.  A chain of n links takes n + 1 launches: link 0's latent kernel,
// n - 1 of these, link n - 1's expand kernel (two per link otherwise).
//
// Latent regions (kChainRegion floats each, one row: t of every branch, then
// the sum of squares of an RMSNorm input): link 0's latent kernel fills
// region 0 and clears the last region (kChainLast, left by the final expand
// of the chain before); the kernel joining links j and j + 1 reads region j,
// fills region j + 1 (the last region when j + 1 = n - 1) and clears region
// j - 1, which the kernel before it read; the final expand reads the last
// region and clears region n - 2.  No kernel clears a region another kernel
// of the chain still reads or fills, and every region but the last is zero
// again when a chain ends, whatever its length.
// ---------------------------------------------------------------------------
constexpr int kMaxChainLinks = 8;
constexpr int kChainRegion = int(kMaxRankTotal) + kMaxSeg * 128 + kSsqSlots;  // floats
constexpr int kChainLast = kMaxChainLinks - 1;  // index of the last region
static_assert(kChainRegion % 64 == 0, "regions keep 256-byte alignment");

// The joined kernel's arguments, compact: every kernel-argument cache line a
// kernel touches first costs a memory round trip, and two full MfmaParams
// (about 2 KB, reached in dependent steps) cost several.
struct ChainProj {  // a projection of link j, as the joined kernel expands it
  const uint32_t* U[2];
  const float* h[2];
  const float* bias;
  const float* res;
  float* y;
  int RW[2];
  int steps[2];  // rank steps (4 sign words each) per branch
  int tbase[2];
  int nb;
  int pad;
};
struct ChainSeg {  // a segment (branch) of link j + 1, as the joined kernel reads it
  const uint32_t* vt;  // V's tiled copy
  const float* l;
  const float* g;
  int R;
  int tbase;
};
struct ChainParams {
  const float* tsrc;  // link j's t, then its sum of squares at tsrc + tsize_e
  float* tdst;        // link j + 1's t, then its sum of squares at tdst + tsize_l
  const float* nw;    // link j + 1's RMSNorm weight
  float* clr;         // cleared here, spread over the blocks
  int tsize_e, late, Ke, N;  // link j: t floats, 1/rms deferred to here, K, outputs
  float eps;
  int nseg, Kl, KWl, xmode, tsize_l, nclr, pad;  // link j + 1
  ChainProj proj[2];
  ChainSeg seg[kMaxSeg];
};

// grid = ceil(N / C) blocks of W waves; wave w expands rows c0 + 16 w .. + 15
// of each projection p < NT (all of its rank steps, both branches), lanes
// 0..15 ending with y of row c0 + 16 w + lane.  LDS: link j's t (compact,
// per projection and branch, 16 chunks of 8 ranks per step), then link
// j + 1's A operand per segment (NCH chunks).
template <int S, int W, int NT>
__global__ __launch_bounds__(W * kWave) void chain_mfma_kernel(ChainParams cp) {
  using L = Compact<1>;
  constexpr int THREADS = W * kWave;
  constexpr int C = 16 * W;   // rows of link j per block = k-chunk of link j + 1
  constexpr int NCH = C / 8;  // 8-column chunks of the k-chunk
  constexpr int NVW = C / 32; // V words per latent row of the k-chunk
  // latent tiles per wave whose V words are in flight at once (16-32 VGPRs)
  constexpr int TPW = NVW <= 4 ? 8 : 2;
  static_assert(NT == 1 || NT == 2, "one projection, or gate and up");
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  u32x4* lds = reinterpret_cast<u32x4*>(lds_raw);
  __shared__ float xs[C];
  __shared__ float ssqw[W];
  const int tid = int(threadIdx.x);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int c0 = int(blockIdx.x) * C;
  // link j + 1's latent stage: wave w takes segment w % nseg (nseg <= W),
  // and of its 16-row tiles those k with k % nws == w / nseg, nws the waves
  // of that segment; the A operand of segment w is built by wave w.  The
  // segment's fields are read here, so that their round trip overlaps the
  // issue of the loads below.
  const int nseg = cp.nseg;
  const int ws = wave % nseg;
  const int wi = wave / nseg;
  const int nws = (W - ws + nseg - 1) / nseg;
  const ChainSeg& G = cp.seg[ws];
  const int ntile = (G.R + 15) >> 4;
  const int N = cp.N;
  const int n = c0 + 16 * wave + col;
  const bool nvalid = n < N;
  const int nc = nvalid ? n : 0;

  // link j's step sequences and staged chunks, (projection, branch) in order
  // (no local array is indexed per lane below: the compiler would keep it in
  // scratch memory)
  StepSeq sq[NT];
  int nchb[2 * NT], cb[2 * NT], tbb[2 * NT];
  int ntask = 0;
#pragma unroll
  for (int q = 0; q < NT; ++q) {
    const ChainProj& P = cp.proj[q];
    const bool two = P.nb > 1;
    sq[q].U[0] = P.U[0];
    sq[q].U[1] = P.U[two ? 1 : 0];
    sq[q].RW[0] = P.RW[0];
    sq[q].RW[1] = P.RW[two ? 1 : 0];
    sq[q].steps[0] = P.steps[0];
    sq[q].steps[1] = P.steps[two ? 1 : 0];
    sq[q].P0 = two ? (sq[q].steps[0] + 3) & ~3 : sq[q].steps[0];
    sq[q].N = N;
    nchb[2 * q] = 16 * sq[q].steps[0];
    nchb[2 * q + 1] = two ? 16 * sq[q].steps[1] : 0;
    tbb[2 * q] = P.tbase[0];
    tbb[2 * q + 1] = P.tbase[two ? 1 : 0];
    cb[2 * q] = ntask;
    ntask += nchb[2 * q];
    cb[2 * q + 1] = ntask;
    ntask += nchb[2 * q + 1];
  }
  const float* __restrict__ ta = cp.tsrc;

  // (1) staging loads of the thread's first task (chunk h: 8 ranks of t)
  const int cb1 = cb[1], tb0 = tbb[0], tb1 = tbb[1];
  const int cb2 = NT == 2 ? cb[2 % (2 * NT)] : ntask, cb3 = NT == 2 ? cb[3 % (2 * NT)] : ntask;
  const int tb2 = NT == 2 ? tbb[2 % (2 * NT)] : 0, tb3 = NT == 2 ? tbb[3 % (2 * NT)] : 0;
  auto src_of = [&](int h) {
    // chunk h - cb[i] of piece i starts at tbb[i] + 8 (h - cb[i])
    const int base = h < cb1 ? tb0 : h < cb2 ? tb1 - 8 * cb1 : h < cb3 ? tb2 - 8 * cb2 : tb3 - 8 * cb3;
    return ta + base + 8 * h;
  };
  float4 v0 = {0.f, 0.f, 0.f, 0.f}, v1 = {0.f, 0.f, 0.f, 0.f};
  if (tid - lane < ntask) {
    const float* s0 = src_of(min(tid, ntask - 1));
    v0 = *reinterpret_cast<const float4*>(s0);
    v1 = *reinterpret_cast<const float4*>(s0 + 4);
  }
  const bool late = cp.late != 0;
  // a vector load (index opaque to the compiler): a scalar one would make
  // every later wait for the kernel arguments wait for it too
  int zero = 0;
  asm volatile("" : "+v"(zero));
  const float ssq = late ? ta[cp.tsize_e + zero] : 0.f;
  auto put = [&](int h, float4 a0, float4 a1, float r) {
    const float a[8] = {a0.x * r, a0.y * r, a0.z * r, a0.w * r, a1.x * r, a1.y * r, a1.z * r, a1.w * r};
    u32x4 hi, lo;
    split8(a, hi, lo);
    u32x4* base = lds + size_t(h) * L::ROWS;
    base[0] = hi;
    base[1] = lo;
    base[2] = u32x4{0u, 0u, 0u, 0u};
  };
  float rs = 1.f;
  // more chunks than threads: all staged here, before the sign words are
  // issued (a loop of loads and waits after them would wait for them too)
  const bool tail = ntask > THREADS;  // block-uniform
  if (tail) {
    if (late) rs = inv_rms(ssq, 1.f / float(cp.Ke), cp.eps);
    if (tid < ntask) put(tid, v0, v1, rs);
    for (int h = tid + THREADS; h < ntask; h += THREADS) {
      const float* s = src_of(h);
      put(h, *reinterpret_cast<const float4*>(s), *reinterpret_cast<const float4*>(s + 4), rs);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // (2) sign words of the wave's rows, every step of each projection
  SignWords<S> sw[NT];
#pragma unroll
  for (int q = 0; q < NT; ++q) sw[q].load(sq[q], nc, 0, sq[q].P0 + (cp.proj[q].nb > 1 ? sq[q].steps[1] : 0), grp);
  // (3) epilogue operands of link j
  float h0v[NT], h1v[NT], bnv[NT], resv[NT];
#pragma unroll
  for (int q = 0; q < NT; ++q) {
    const ChainProj& P = cp.proj[q];
    h0v[q] = P.h[0][nc];
    h1v[q] = P.nb > 1 ? P.h[1][nc] : 0.f;
    bnv[q] = P.bias ? P.bias[nc] : 0.f;
    resv[q] = P.res ? P.res[nc] : 0.f;
  }
  // link j + 1's RMSNorm weight at k = n, before the V words below (waits
  // retire in issue order: a load after them would wait for them)
  const float nwv = cp.xmode == LBK_INPUT_RMSNORM ? cp.nw[nc] : 1.f;
  // (4) link j + 1's latent stage (its segment's fields were read first)
  const int kw0 = c0 / 32;
  const int kw4 = (cp.KWl + 3) >> 2;
  // V words of the k-chunk for the lane's row of the wave's k-th tile, from
  // V's tiled copy [ceil(R/16)][ceil(KW/4)][16 rows][4 words] (whole 16-byte
  // cells), and l of the row
  auto load_vw = [&](int k, uint32_t (&w)[NVW], float& lv) {
    const int t = min(wi + k * nws, ntile - 1);
    const int r = 16 * t + col;
    const int rr = r < G.R ? r : 0;
    lv = G.l[rr];
    const uint32_t* __restrict__ cells = G.vt + size_t(rr >> 4) * kw4 * 64 + (rr & 15) * 4;
    if constexpr (NVW == 2) {
      const int gi = kw0 < cp.KWl ? kw0 >> 2 : 0;
      const uint2 v = *reinterpret_cast<const uint2*>(cells + size_t(gi) * 64 + (kw0 & 3));
      w[0] = v.x;
      w[1] = v.y;
    } else {
#pragma unroll
      for (int q = 0; q < NVW / 4; ++q) {
        const int gi = (kw0 >> 2) + q < kw4 ? (kw0 >> 2) + q : 0;
        const uint4 v = *reinterpret_cast<const uint4*>(cells + size_t(gi) * 64);
        w[4 * q] = v.x;
        w[4 * q + 1] = v.y;
        w[4 * q + 2] = v.z;
        w[4 * q + 3] = v.w;
      }
    }
  };
  // g of the A operand (lanes < NCH one 8-column chunk each; masked where
  // used: a use here would wait for every load issued before it), before
  // the V words, which the A operand's wait then does not cover
  const int ac = lane;
  const int ak = c0 + 8 * ac;
  const bool gin = wave < nseg && ac < NCH && ak < cp.Kl;  // K % 8 == 0: wholly inside or past K
  Raw8<float> g8;
  g8.load(G.g + (gin ? ak : 0));
  // the V words of the wave's first TPW tiles (those it has): one round trip
  // for them all
  uint32_t vw[TPW][NVW];
  float lv[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i)
    if (wi + i * nws < ntile) load_vw(i, vw[i], lv[i]);
  // (5) the region this launch clears
  {
    const int nblk = int(gridDim.x), bl = int(blockIdx.x);
    const int per = (cp.nclr + nblk - 1) / nblk;
    const int hi = min(cp.nclr, (bl + 1) * per);
    for (int i = bl * per + tid; i < hi; i += THREADS) cp.clr[i] = 0.f;
  }
  __builtin_amdgcn_sched_barrier(0);
  if (!tail) {
    if (late) rs = inv_rms(ssq, 1.f / float(cp.Ke), cp.eps);
    if (tid < ntask) put(tid, v0, v1, rs);
  }
  __syncthreads();

  // (6) expand: y of the lane's row for each projection
  uint32_t kmask = 0x80008000u, kone = 0x3F803F80u;
  asm volatile("" : "+v"(kmask), "+v"(kone));
  const int lrow = L::lane_row(col);
  float y[NT];
#pragma unroll
  for (int q = 0; q < NT; ++q) {
    const u32x4* __restrict__ tb0 = lds + size_t(cb[2 * q]) * L::ROWS;
    const u32x4* __restrict__ tb1 = lds + size_t(cb[2 * q + 1]) * L::ROWS;
    const bool two = cp.proj[q].nb > 1;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f}, acc0 = {0.f, 0.f, 0.f, 0.f};
    bool in1 = false;
    auto enter = [&](bool b1) {
      if (b1 && !in1) {
        acc0 = acc;
        acc = f32x4{0.f, 0.f, 0.f, 0.f};
        in1 = true;
      }
    };
    auto mfma4 = [&](uint32_t word, const u32x4* __restrict__ tb, int w, uint32_t km, uint32_t ko) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x8 bop = signs_to_bf16x8(word, j, km, ko);
        const bf16x8 aop = __builtin_bit_cast(bf16x8, tb[(4 * w + j) * L::ROWS + lrow]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop, acc, 0, 0, 0);
      }
    };
    const int nst = sq[q].P0 + (two ? sq[q].steps[1] : 0);
    const int G = nst >> 2, rem = nst & 3;
#pragma unroll
    for (int t = 0; t < S / 4; ++t) {
      if (t >= G) continue;
      const bool b1 = 4 * t >= sq[q].P0;
      enter(b1);
      uint32_t w4[4];
      sw[q].group(t, w4);
      // steps in branch 0's padding get a zero B operand
      const int st = (b1 ? 4 * t - sq[q].P0 : 4 * t) + grp;
      const bool valid = b1 || st < sq[q].steps[0];
      const int sv = valid ? st : 0;
      const uint32_t km = valid ? kmask : 0u, ko = valid ? kone : 0u;
#pragma unroll
      for (int u = 0; u < 4; ++u) mfma4(w4[u], b1 ? tb1 : tb0, 4 * sv + u, km, ko);
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (i >= rem) continue;
      const int qs = 4 * G + i;
      const bool b1 = qs >= sq[q].P0;
      enter(b1);
      mfma4(sw[q].rem[i], b1 ? tb1 : tb0, 4 * (b1 ? qs - sq[q].P0 : qs) + grp, kmask, kone);
    }
    if (!in1) {
      acc0 = acc;
      acc = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // C row 0 (lanes 0..15) is hi of the row, C row 8 (lanes 32..47) lo
    const float s0 = add_upper32(acc0[0]);
    const float s1 = add_upper32(acc[0]);
    y[q] = h0v[q] * s0 + h1v[q] * s1 + bnv[q] + resv[q];
  }
  // (7) link j's outputs, and link j + 1's input at k = n
  float xv = 0.f;
  if (lane < 16) {
#pragma unroll
    for (int q = 0; q < NT; ++q)
      if (nvalid) cp.proj[q].y[n] = y[q];
    if (nvalid) {
      if constexpr (NT == 2) xv = silu_f(y[0]) * y[1];
      else xv = cp.xmode == LBK_INPUT_RMSNORM ? y[0] * nwv : y[0];
    }
    xs[16 * wave + col] = xv;
  }
  if (cp.xmode == LBK_INPUT_RMSNORM) {
    // the rows' sum of squares: lanes 0..15 of each wave, then the block
    const float q2 = row16_sum(lane < 16 && nvalid ? y[0] * y[0] : 0.f);
    if (lane == 0) ssqw[wave] = q2;
  }
  __syncthreads();
  if (cp.xmode == LBK_INPUT_RMSNORM && tid == 0) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) s += ssqw[w];
    unsafeAtomicAdd(cp.tdst + cp.tsize_l, s);
  }
  // (8) A operand of link j + 1: hi / lo of g[k] * x[k], segment w by wave w
  u32x4* lds_a = lds + size_t(ntask) * L::ROWS;
  if (wave < nseg && ac < NCH) {
    float gv[8], a[8];
    g8.get(gv);
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = gv[e] * xs[8 * ac + e];
    if (!gin) {
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = 0.f;
    }
    u32x4 hi, lo;
    split8(a, hi, lo);
    u32x4* base = lds_a + size_t(wave * NCH + ac) * L::ROWS;
    base[0] = hi;
    base[1] = lo;
    base[2] = u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();

  // (9) the wave's latent tiles in batches of TPW: NVW MFMAs each over the
  // k-chunk, then one fp32 atomic per latent row
  // the segment's A operand: the same NVW fragments for every tile
  bf16x8 aop[NVW];
#pragma unroll
  for (int kk = 0; kk < NVW; ++kk)
    aop[kk] = __builtin_bit_cast(bf16x8, lds_a[(size_t(ws) * NCH + 4 * kk + grp) * L::ROWS + lrow]);
  for (int k0 = 0; k0 * nws + wi < ntile; k0 += TPW) {
    if (k0 > 0) {
#pragma unroll
      for (int i = 0; i < TPW; ++i)
        if (wi + (k0 + i) * nws < ntile) load_vw(k0 + i, vw[i], lv[i]);
    }
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int t = wi + (k0 + i) * nws;
      if (t >= ntile) continue;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NVW; ++kk) {
        const bf16x8 bop = signs_to_bf16x8(vw[i][kk], grp, kmask, kone);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[kk], bop, acc, 0, 0, 0);
      }
      const float sum = add_upper32(acc[0]);
      const int r = 16 * t + col;
      if (lane < 16 && r < G.R) unsafeAtomicAdd(cp.tdst + G.tbase + r, lv[i] * sum);
    }
  }
}

// ---------------------------------------------------------------------------
// GEMM path (M > 16, and shapes the decode path cannot stage in LDS): a
// tiled sign-GEMM on v_mfma_f32_32x32x16_bf16, three launches per call.
//   prologue  A_s[m, k] = g_s[k] * x[m, k] per branch s, as bf16, k padded
//             with zeros to a multiple of 64
//   stage 1   T_s[m, r] = l_s[r] * sum_k sV_s[r, k] * A_s[m, k], as bf16
//   stage 2   y[m, n] = bias[n] + sum_b h_b[n] * sum_r sU_b[n, r] * T_b[m, r]
// With SPLIT (fp32 activations) A and T are stored as two bf16 planes, hi
// and lo = bf16(v - hi), and both planes go through the MFMA, so products
// keep ~2^-17 relative error.  Without SPLIT (bf16 activations) one plane:
// the precision of the reference's bf16 forward (littlebit.py:116-121).
// Stages 1 and 2: block tile 128 (m) x 128 (columns: latent rows in stage
// 1, outputs in stage 2), 4 waves of 64 x 64 (2 x 2 MFMA tiles), k-steps of
// 64.  A tiles go from global memory straight to LDS through a 4-stage ring
// (see gemm_mainloop); the +-1 B operand is expanded in registers from the
// sign words of the lane's column (staged in LDS by the block): for 16-k
// sub-step s, lane l (column l % 32, k 8*(l/32) .. +8 of the 32x32x16
// operand) takes byte 2*(s%2) + l/32 of word s/2 of the step.
// ---------------------------------------------------------------------------
constexpr int kGB = 128;             // block tile (m and columns)
constexpr int kGK = 64;              // k per step (two sign words per column)
constexpr int kGThreads = 256;

typedef float f32x16 __attribute__((ext_vector_type(16)));

struct GemmSeg {      // stage-1 operands of one branch
  const uint32_t* V;  // [R, KW]
  const float* g;     // [K]
  const float* l;     // [R]
  int R;
  int RP;             // T row length: R rounded up to kGB
  int nt0;            // first column tile of the segment
  int64_t abase;      // offset of the segment's [M][Kp] block in an A plane
  int64_t tbase;      // offset of the segment's [M][RP] block in a T plane
};

struct GemmProj {     // stage-2 operands of one projection
  const uint32_t* U[2];
  const float* h[2];
  const float* bias;
  const float* res;   // [M, N] fp32 added to y, or null (may alias y)
  void* y;
  int RW[2];          // words per U row
  int RP[2];
  int64_t tbase[2];
  int nb;
  int N;
  int nt0;            // first column tile of the projection
};

struct GemmParams {
  GemmSeg seg[kMaxSeg];
  GemmProj proj[kMaxProj];
  int nseg, nproj;
  int M, K, KW;
  int Kp;             // K rounded up to kGK
  int xvec;           // x rows (x1, rms weight) and every g allow 16-byte loads
  int xmode;          // LBK_INPUT_* (see load_input8)
  const void* x;
  const void* x1;
  const float* nw;
  float eps;
  uint16_t* a;        // A planes (hi, then lo with SPLIT)
  uint16_t* t;        // T planes
  int64_t a_plane;    // elements per A plane
  int64_t t_plane;    // elements per T plane
};

// hi = bf16(v), lo = bf16(v - hi), round to nearest even
__device__ __forceinline__ void split1(float v, uint16_t& hi, uint16_t& lo) {
  hi = f32_to_bf16(v);
  lo = f32_to_bf16(v - bf16_to_f32(hi));
}

// Prologue.  grid = (M, segments), 256 threads; thread handles 8-k chunks.
// The input mode (RMSNorm, SiLU * up) is applied here, as in load_input8.
template <typename XT, bool SPLIT>
__global__ __launch_bounds__(kGThreads) void gemm_scale_kernel(GemmParams p) {
  const int m = int(blockIdx.x);
  const GemmSeg& S = p.seg[__builtin_amdgcn_readfirstlane(int(blockIdx.y))];
  const XT* __restrict__ xr = static_cast<const XT*>(p.x) + int64_t(m) * p.K;
  const XT* __restrict__ ur = p.x1 ? static_cast<const XT*>(p.x1) + int64_t(m) * p.K : xr;
  const float* __restrict__ g = S.g;
  const int tid = int(threadIdx.x);
  float rsm = 1.f;
  if (p.xmode == LBK_INPUT_RMSNORM) {
    __shared__ float rs[1];
    __shared__ float rscratch[kGThreads / 64];
    rms_scales<XT, 1, kGThreads>(xr, 1, p.K, p.eps, rs, rscratch, tid);
    rsm = rs[0];
  }
  uint16_t* __restrict__ hi = p.a + S.abase + int64_t(m) * p.Kp;
  for (int k = 8 * tid; k < p.Kp; k += 8 * kGThreads) {
    float v[8];
    if (p.xvec && k + 8 <= p.K) {
      float gv[8];
      load8(xr + k, v);
      load8(g + k, gv);
      if (p.xmode == LBK_INPUT_RMSNORM) {
        float wv[8];
        load8(p.nw + k, wv);
#pragma unroll
        for (int i = 0; i < 8; ++i) gv[i] *= wv[i] * rsm;
      } else if (p.xmode == LBK_INPUT_SILU_MUL) {
        float uv[8];
        load8(ur + k, uv);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = silu_f(v[i]) * uv[i];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] *= gv[i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float e = 0.f;
        if (k + i < p.K) {
          const float xv = to_f32(xr[k + i]);
          e = xv * g[k + i];
          if (p.xmode == LBK_INPUT_RMSNORM) e *= p.nw[k + i] * rsm;
          else if (p.xmode == LBK_INPUT_SILU_MUL) e = silu_f(xv) * to_f32(ur[k + i]) * g[k + i];
        }
        v[i] = e;
      }
    }
    if constexpr (SPLIT) {
      u32x4 h, l;
      split8(v, h, l);
      *reinterpret_cast<u32x4*>(hi + k) = h;
      *reinterpret_cast<u32x4*>(hi + p.a_plane + k) = l;
    } else {
      u32x4 h;
#pragma unroll
      for (int d = 0; d < 4; ++d) h[d] = uint32_t(f32_to_bf16(v[2 * d])) | (uint32_t(f32_to_bf16(v[2 * d + 1])) << 16);
      *reinterpret_cast<u32x4*>(hi + k) = h;
    }
  }
}

// acc[i][j] += A[m0 + gemm_row(wm, i) + .., :64*nks] . S[:64*nks, c0 + gemm_col<NJ>(wn, j) + ..]
// S[k, c] = sign bit k of row c of W (ldw words per row, zero past it);
// step ks reads words 2*ks and 2*ks + 1.  The block covers 128 rows of A and
// BN = 128 or 256 columns (wide: each staged A tile serves twice the
// columns), its 4 waves laid out as below.
//
// A tiles (128 rows x 64 k per plane, rows past M repeat row M - 1) go from
// global memory straight to LDS (global_load_lds_dwordx4) through a ring of
// kGStages stages, issued kGStages - 1 steps ahead; each stage is its own
// __shared__ array so that the compiler can tell which load fills which
// stage.  Rows are 128 bytes, 16-byte chunk c of row r stored at chunk
// c ^ swz(r), swz(r) = (r ^ (r >> 3)) & 7: the LDS serves a ds_read_b128 16
// lanes (256 bytes, all 64 banks) at a time, and the 16 rows of such a group
// -- 8 of each row parity, at the same offset mod 256 -- read 16 distinct
// 16-byte bank groups (with c ^ (r & 7), rows r and r + 8 collided).
//
// The sign words of a step (2 per column, BN columns) are fetched by the
// whole block, BN / 128 words per thread (columns 128 u + tid / 2, word
// tid % 2), and written to one of two LDS buffers ([column][2 words]) from
// which every lane of the step reads its columns' pair (8 bytes).  A lane fetching
// its own columns' words instead costs 16 loads per block and step, each
// touching 32 cache lines, and the two wave rows fetch the same words.
//
// With GB (stage 1 on bf16 activations taken as they are) the B operand is
// +-g[k] instead of +-1: the 64 g values of a step are staged beside its
// sign words, as bf16, in one of two 128-byte buffers (each wave fetches
// them, wave 0 writes them), and each 16-k sub-step reads its 8 values.
// In wide tiles (BN = 256) with h given (the second branch of stage 2, h0 the
// first branch's row scale) it is +-1 where the lane's column c keeps
// branch 1 (use_branch1(h0[c], h[c])) and 0 elsewhere; both branches run
// the same instantiation, so they share one stage ring.
//
// fill(f) issues the DMA of step f and the sign word (and g) of step f + 1.  Every
// fill issues the same loads on every path; before step ks every wave waits
// (vmcnt) until only the two newer fills' loads are outstanding -- vector
// loads complete in order, so fill(ks) has landed: stage ks is complete and
// the sign word of step ks + 1 is in the register that step ks writes to LDS
// (masked to zero past the row or the matrix) -- and a barrier makes the
// tile, and the words step ks - 1 wrote, visible; fill(ks + 3) then refills
// the stage and the register that step ks - 1 used.  Ends with a barrier.
[[maybe_unused]] constexpr int kGStages = 4;  // the ring's stages (one __shared__ array each)

// Wave layout of a GEMM block: kGWM waves along m, kGWN along the columns;
// a wave holds kGMI x NJ tiles of 32 x 32 (NJ = BN / (32 kGWN)).  The B
// operand is expanded in registers from the sign words, once per wave for
// each of its column tiles, and feeds the kGMI MFMAs of that column; each A
// fragment read from LDS feeds NJ.  Tall wave tiles (kGWM = 1: all 128 rows,
// 4 x 1 tiles at BN = 128, 4 x 2 at BN = 256) expand each sign once per
// block, half the VALU per MFMA of 2 x 2 waves, and read each A fragment for
// NJ MFMAs instead of 2 NJ: measured, MFMAs fed from LDS lose about 1 % at
// one fragment per MFMA, while VALU beyond about 4 per MFMA stalls the MFMA
// pipe (bench.py --only issue).
#ifndef LBK_GEMM_WM
#define LBK_GEMM_WM 1
#endif
constexpr int kGWM = LBK_GEMM_WM;
constexpr int kGWN = 4 / kGWM;
constexpr int kGMI = kGB / (32 * kGWM);
static_assert(kGWM == 1 || kGWM == 2, "wave layouts 1 x 4 and 2 x 2");
template <int BN>
constexpr int gemm_nj() {
  return BN / (32 * kGWN);
}
__device__ __forceinline__ int gemm_row(int wm, int i) { return 32 * kGMI * wm + 32 * i; }
template <int NJ>
__device__ __forceinline__ int gemm_col(int wn, int j) {
  return 32 * NJ * wn + 32 * j;
}
__device__ __forceinline__ int gemm_wm(int wave) { return kGWM == 1 ? 0 : wave >> 1; }
__device__ __forceinline__ int gemm_wn(int wave) { return kGWM == 1 ? wave : wave & 1; }

template <bool SPLIT, bool GB = false, int BN = 128>
__device__ __forceinline__ void gemm_mainloop(const uint16_t* __restrict__ A, int64_t plane, int64_t lda, int M,
                                              int m0, const uint32_t* __restrict__ W, int ldw, int ncols, int c0,
                                              int nks, f32x16 (&acc)[kGMI][gemm_nj<BN>()], int tid,
                                              const float* __restrict__ g = nullptr, int kbase = 0,
                                              const float* __restrict__ h = nullptr,
                                              const float* __restrict__ h0 = nullptr) {
  static_assert(BN == 128 || BN == 256, "blocks of 128 or 256 columns");
  static_assert(BN == 128 || !GB, "wide tiles carry no g in the B operand");
  constexpr int NJ = gemm_nj<BN>();
  typedef __attribute__((address_space(3))) void* lds_ptr_t;
  typedef __attribute__((address_space(1))) void* glb_ptr_t;
  constexpr int NT = SPLIT ? 2 : 1;
  constexpr int NW = BN / 128;              // sign words per thread and step
  constexpr int TILE = kGB * kGK;           // elements per plane per stage
  constexpr int LOADS_PER_FILL = 4 * NT + NW + (GB ? 1 : 0);  // global_load_lds, sign words, g; per wave
  __shared__ __attribute__((aligned(16))) uint16_t st0[NT * TILE];
  __shared__ __attribute__((aligned(16))) uint16_t st1[NT * TILE];
  __shared__ __attribute__((aligned(16))) uint16_t st2[NT * TILE];
  __shared__ __attribute__((aligned(16))) uint16_t st3[NT * TILE];
  __shared__ __attribute__((aligned(16))) uint32_t sw[2][2 * BN];
  __shared__ __attribute__((aligned(16))) uint16_t gb[2][kGK];
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = gemm_wm(wave), wn = gemm_wn(wave);
  const int lr = lane & 31, lh = lane >> 5;
  // Steps are numbered from kbase (the first k-step of the range, 64 k
  // each); step st of the range is k-step kbase + st of the matrices.
  // this thread's sign words of a step: word 2 * step + (tid & 1) of
  // columns c0 + 128 u + tid / 2, stored at sw[.][2 * (128 u + tid / 2) + tid % 2]
  const int sodd = tid & 1;
  uint32_t smask[NW];
  const uint32_t* __restrict__ srow[NW];
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    const int scol = c0 + 128 * u + (tid >> 1);
    smask[u] = scol < ncols ? ~0u : 0u;
    srow[u] = W + int64_t(scol < ncols ? scol : 0) * ldw;
  }
  struct Words {
    uint32_t v[NW];
  };
  auto word_at = [&](int st) {
    Words w;
#pragma unroll
    for (int u = 0; u < NW; ++u) w.v[u] = srow[u][min(2 * (kbase + st) + sodd, ldw - 1)];
    return w;
  };
  // The empty asm pins each register's first use to its step: without it
  // the compiler hoists the masking of later steps' words into this one and
  // waits there for every outstanding load (vmcnt(0)), DMAs included.
  auto put_word = [&](int st, Words raw) {
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      uint32_t r = raw.v[u];
      asm volatile("" : "+v"(r));
      sw[st & 1][256 * u + tid] = 2 * (kbase + st) + sodd < ldw ? r & smask[u] : 0u;
    }
  };
  // wide tiles: the +-1 pair of the lane's column in subtile j, or 0 where
  // h is given and the column drops branch 1 (columns past ncols have zero
  // sign words)
  uint32_t hv[NJ];
  if constexpr (BN == 256) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = min(c0 + gemm_col<NJ>(wn, j) + lr, ncols - 1);
      hv[j] = !h || use_branch1(h0[n], h[n]) ? 0x3F803F80u : 0u;
    }
  }
  // g of step st, lane's k (clamped: steps past the last are never read)
  const int kmax = (kbase + nks) * kGK - 1;
  auto g_at = [&](int st) { return GB ? g[min((kbase + st) * kGK + lane, kmax)] : 0.f; };
  auto put_g = [&](int st, float v) {
    if constexpr (GB) {
      asm volatile("" : "+v"(v));
      if (wave == 0) gb[st & 1][lane] = f32_to_bf16(v);
    }
  };
  // this lane's source rows and chunks for its 4 DMA slots of a stage
  const uint16_t* src[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int slot = (wave * 4 + j) * 64 + lane;
    const int row = slot >> 3, c = (slot & 7) ^ ((row ^ (row >> 3)) & 7);
    src[j] = A + int64_t(min(m0 + row, M - 1)) * lda + 8 * c;
  }
  auto issue = [&](int ks, uint16_t* st) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint16_t* dst = st + (wave * 4 + j) * 512;
      __builtin_amdgcn_global_load_lds((glb_ptr_t)(src[j] + int64_t(kbase + ks) * kGK), (lds_ptr_t)dst, 16, 0, 0);
      if constexpr (SPLIT)
        __builtin_amdgcn_global_load_lds((glb_ptr_t)(src[j] + plane + int64_t(kbase + ks) * kGK), (lds_ptr_t)(dst + TILE),
                                         16, 0, 0);
    }
  };
  uint32_t kmask = 0x80008000u, kone = 0x3F803F80u;
  asm volatile("" : "+v"(kmask), "+v"(kone));
  auto compute = [&](int ks, const uint16_t* a) {
    u32x4 gk[4];
    if constexpr (GB) {
#pragma unroll
      for (int s = 0; s < 4; ++s) gk[s] = *reinterpret_cast<const u32x4*>(&gb[ks & 1][16 * s + 8 * lh]);
    }
    uint32_t w[NJ][2];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint2 pr = *reinterpret_cast<const uint2*>(&sw[ks & 1][2 * (gemm_col<NJ>(wn, j) + lr)]);
      w[j][0] = pr.x;
      w[j][1] = pr.y;
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8 b[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        b[j] = GB   ? signs_times_bf16x8(w[j][s >> 1] >> (8 * lh), 2 * (s & 1), kmask, gk[s])
               : BN == 256 ? signs_times_bf16x8(w[j][s >> 1] >> (8 * lh), 2 * (s & 1), kmask,
                                               u32x4{hv[j], hv[j], hv[j], hv[j]})
                    : signs_to_bf16x8(w[j][s >> 1] >> (8 * lh), 2 * (s & 1), kmask, kone);
#pragma unroll
      for (int i = 0; i < kGMI; ++i) {
        const int r = gemm_row(wm, i) + lr;
        const int off = r * kGK + (((2 * s + lh) ^ ((r ^ (r >> 3)) & 7)) << 3);
        const bf16x8 ah = *reinterpret_cast<const bf16x8*>(a + off);
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, b[j], acc[i][j], 0, 0, 0);
        if constexpr (SPLIT) {
          const bf16x8 al = *reinterpret_cast<const bf16x8*>(a + TILE + off);
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, b[j], acc[i][j], 0, 0, 0);
        }
      }
    }
  };
  // Past the last step a fill repeats step nks - 1's DMA into a stage nothing
  // reads again (and a clamped word nothing reads), so exactly two fills'
  // loads are always newer than fill(ks) at step ks.
  auto fill = [&](int f, uint16_t* st, Words& w, float& gv) {
    w = word_at(f + 1);
    gv = g_at(f + 1);
    issue(min(f, nks - 1), st);
  };
  // The memory clobbers keep LDS accesses from being moved across the
  // barrier; the waitcnt and the barrier also delimit the scheduler's
  // regions, so fills ks + 1 and ks + 2 issue all their loads after fill ks.
  auto step = [&](int ks, const uint16_t* cur, Words wcur, float gcur, uint16_t* nxt, Words& wnxt,
                  float& gnxt) {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(2 * LOADS_PER_FILL));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    put_word(ks + 1, wcur);
    put_g(ks + 1, gcur);
    fill(ks + 3, nxt, wnxt, gnxt);
    compute(ks, cur);
  };
  put_word(0, word_at(0));
  put_g(0, g_at(0));
  Words w0, w1, w2, w3;
  float g0, g1, g2, g3;
  fill(0, st0, w0, g0);
  __builtin_amdgcn_sched_barrier(0);
  fill(1, st1, w1, g1);
  __builtin_amdgcn_sched_barrier(0);
  fill(2, st2, w2, g2);
  __builtin_amdgcn_sched_barrier(0);
  // whole rounds of the ring, then the remaining steps: every path into the
  // loop header has issued the same loads
  int ks = 0;
  for (; ks + 4 <= nks; ks += 4) {
    step(ks, st0, w0, g0, st3, w3, g3);
    step(ks + 1, st1, w1, g1, st0, w0, g0);
    step(ks + 2, st2, w2, g2, st1, w1, g1);
    step(ks + 3, st3, w3, g3, st2, w2, g2);
  }
  if (ks < nks) step(ks, st0, w0, g0, st3, w3, g3);
  if (ks + 1 < nks) step(ks + 1, st1, w1, g1, st0, w0, g0);
  if (ks + 2 < nks) step(ks + 2, st2, w2, g2, st1, w1, g1);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Stage 1 epilogue: T rows of the tile (m0, c0) of segment G, l-scaled.
constexpr int kGNJ = gemm_nj<kGB>();  // column tiles per wave of a 128-column block

template <bool SPLIT>
__device__ __forceinline__ void latent_store(const GemmParams& p, const GemmSeg& G, int m0, int c0,
                                             const f32x16 (&acc)[kGMI][kGNJ], int tid) {
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = gemm_wm(wave), wn = gemm_wn(wave);
  const int lr = lane & 31, lh = lane >> 5;
  uint16_t* __restrict__ T = p.t + G.tbase;
#pragma unroll
  for (int j = 0; j < kGNJ; ++j) {
    const int r = c0 + gemm_col<kGNJ>(wn, j) + lr;  // < RP; rows R <= r < RP are written as zeros
    const float lv = r < G.R ? G.l[r] : 0.f;
#pragma unroll
    for (int i = 0; i < kGMI; ++i)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int m = m0 + gemm_row(wm, i) + 8 * (q >> 2) + 4 * lh + (q & 3);
        if (m < p.M) {
          const int64_t o = int64_t(m) * G.RP + r;
          const float v = lv * acc[i][j][q];
          if constexpr (SPLIT) {
            uint16_t h, l;
            split1(v, h, l);
            T[o] = h;
            T[p.t_plane + o] = l;
          } else {
            T[o] = f32_to_bf16(v);
          }
        }
      }
  }
}

__device__ __forceinline__ int latent_segment(const GemmParams& p, int nt) {
  int si = 0;
#pragma unroll
  for (int i = 1; i < kMaxSeg; ++i) si += (i < p.nseg && nt >= p.seg[i].nt0) ? 1 : 0;
  return __builtin_amdgcn_readfirstlane(si);
}

// Stage 1.  grid = (m-tiles, column tiles of all segments), 256 threads.
// GB: A is the bf16 input itself (every segment's abase 0, rows of Kp = K)
// and g goes into the B operand.
template <bool SPLIT, bool GB>
__global__ __launch_bounds__(kGThreads) void gemm_latent_kernel(GemmParams p) {
  const int tid = int(threadIdx.x);
  const int nt = int(blockIdx.y);
  const GemmSeg& G = p.seg[latent_segment(p, nt)];
  const int m0 = int(blockIdx.x) * kGB;
  const int c0 = (nt - G.nt0) * kGB;
  f32x16 acc[kGMI][kGNJ];
#pragma unroll
  for (int i = 0; i < kGMI; ++i)
#pragma unroll
    for (int j = 0; j < kGNJ; ++j) acc[i][j] = f32x16{};
  gemm_mainloop<SPLIT, GB>(p.a + G.abase, p.a_plane, p.Kp, p.M, m0, G.V, p.KW, G.R, c0, p.Kp / kGK, acc, tid, G.g);
  latent_store<SPLIT>(p, G, m0, c0, acc, tid);
}

// Stage 1, stream-K form: when the tiles do not fill the CUs' block slots
// evenly (e.g. 272 tiles for 512 slots), resident blocks share the (tile,
// k-step) iterations evenly instead.  The blocks form G groups (G = 8 when
// the m-tiles divide by 8, else 1); group x = b % G takes the tiles of
// m-tiles x, x + G, ... -- blocks are dealt to the 8 XCDs in turn, so each
// XCD's L2 holds the rows of A of two m-tiles (at M = 2048), as in the
// whole-tile grid -- and block b of the group's P blocks (b = blockIdx / G)
// takes its iterations [b W / P, (b + 1) W / P), W = the group's tiles *
// nks, tiles in m-major order.  A tile cut between blocks is
// summed by its last part: every part stores its fp32 accumulators in its
// block's slot (0: the part starts inside the tile, 1: it starts at the
// tile's first step) and adds its step count to the tile's counter (indexed
// by the first block of the tile: each block is the first of at most one cut
// tile); the part whose count completes the tile sums all the parts' slots
// in block order (the same sum on every run), zeroes the counter again and
// stores T.  No part waits for another.
// Partial tiles move through agent-scope stores and loads (sc1: written
// through to, and read from, the point where all XCDs' L2s agree), ordered
// by vmcnt(0) before the counter's atomic; fences would do the same by
// writing back and invalidating whole L2s, which cost more than the tiles.
struct SkParams {
  int P;             // blocks per group
  int G;             // groups (grid = G * P blocks)
  int NT;            // column tiles over all segments
  int nks;           // k-steps per tile
  int64_t W;         // iterations per group: m-tiles / G * NT * nks
  float* part;       // [G * P][2][64 * kGThreads] fp32 partial tiles
  uint32_t* cnt;     // [G * P] step counters, zero between calls
};

__device__ __forceinline__ int64_t sk_start(int b, const SkParams& q) { return int64_t(b) * q.W / q.P; }
// the block whose range holds iteration i: the largest b with sk_start(b) <= i
__device__ __forceinline__ int sk_block(int64_t i, const SkParams& q) { return int(((i + 1) * q.P - 1) / q.W); }

// Two blocks per CU (the sk_blocks plan assumes them): held to 256 registers
// per lane (unbounded, the partial-tile code took 256 VGPRs + 64 AGPRs).
template <bool SPLIT, bool GB>
__global__ __launch_bounds__(kGThreads, 2) void gemm_latent_sk_kernel(GemmParams p, SkParams q) {
  const int tid = int(threadIdx.x);
  const int grp = int(blockIdx.x) % q.G;
  const int b = int(blockIdx.x) / q.G;
  const int gb0 = grp * q.P;  // the group's first slot and counter
  const int64_t it1 = sk_start(b + 1, q);
  __shared__ int s_last;
  for (int64_t it = sk_start(b, q); it < it1;) {
    const int t = int(it / q.nks);
    const int k0 = int(it - int64_t(t) * q.nks);
    const int n = int(min<int64_t>(q.nks - k0, it1 - it));
    const int nt = t % q.NT;
    const GemmSeg& G = p.seg[latent_segment(p, nt)];
    const int m0 = ((t / q.NT) * q.G + grp) * kGB;
    const int c0 = (nt - G.nt0) * kGB;
    f32x16 acc[kGMI][kGNJ];
#pragma unroll
    for (int i = 0; i < kGMI; ++i)
#pragma unroll
      for (int j = 0; j < kGNJ; ++j) acc[i][j] = f32x16{};
    gemm_mainloop<SPLIT, GB>(p.a + G.abase, p.a_plane, p.Kp, p.M, m0, G.V, p.KW, G.R, c0, n, acc, tid, G.g, k0);
    bool store = true;
    if (n < q.nks) {
      const int64_t ts = int64_t(t) * q.nks;
      const int bf = sk_block(ts, q);
      float* __restrict__ mine = q.part + (size_t(gb0 + b) * 2 + (k0 > 0 ? 0 : 1)) * (64 * kGThreads);
#pragma unroll
      for (int i = 0; i < kGMI; ++i)
#pragma unroll
        for (int j = 0; j < kGNJ; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            __hip_atomic_store(mine + ((i * kGNJ + j) * 16 + e) * kGThreads + tid, acc[i][j][e], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
      __syncthreads();
      if (tid == 0) {
        const uint32_t before = __hip_atomic_fetch_add(q.cnt + gb0 + bf, uint32_t(n), __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
        s_last = before + uint32_t(n) == uint32_t(q.nks) ? 1 : 0;
      }
      __syncthreads();
      store = s_last != 0;
      if (store) {
        // the stored parts (this block's too) in block order, whichever
        // block completes the tile: the sum is the same on every run
        const int bl = sk_block(ts + q.nks - 1, q);
#pragma unroll
        for (int i = 0; i < kGMI; ++i)
#pragma unroll
          for (int j = 0; j < kGNJ; ++j) acc[i][j] = f32x16{};
        for (int o = bf; o <= bl; ++o) {
          float* __restrict__ part =
              q.part + (size_t(gb0 + o) * 2 + (sk_start(o, q) > ts ? 0 : 1)) * (64 * kGThreads);
#pragma unroll
          for (int i = 0; i < kGMI; ++i)
#pragma unroll
            for (int j = 0; j < kGNJ; ++j)
#pragma unroll
              for (int e = 0; e < 16; ++e)
                acc[i][j][e] += __hip_atomic_load(part + ((i * kGNJ + j) * 16 + e) * kGThreads + tid, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        }
        if (tid == 0) __hip_atomic_store(q.cnt + gb0 + bf, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (store) latent_store<SPLIT>(p, G, m0, c0, acc, tid);
    it += n;
  }
}

// Stage 2.  grid = (m-tiles, column tiles of all projections), 256 threads.
// Held to 256 registers per lane (two waves per SIMD; unbounded, the two
// accumulator sets took 244 VGPRs + 64 AGPRs, one wave per SIMD).
template <typename YT, bool SPLIT>
__global__ __launch_bounds__(kGThreads, 2) void gemm_expand_kernel(GemmParams p) {
  const int tid = int(threadIdx.x);
  const int nt = int(blockIdx.y);
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxProj; ++i) pi += (i < p.nproj && nt >= p.proj[i].nt0) ? 1 : 0;
  pi = __builtin_amdgcn_readfirstlane(pi);
  const GemmProj& P = p.proj[pi];
  const int m0 = int(blockIdx.x) * kGB;
  const int c0 = (nt - P.nt0) * kGB;
  f32x16 acc0[kGMI][kGNJ], acc1[kGMI][kGNJ];
#pragma unroll
  for (int i = 0; i < kGMI; ++i)
#pragma unroll
    for (int j = 0; j < kGNJ; ++j) acc0[i][j] = acc1[i][j] = f32x16{};
  // T rows are zero from R to RP >= 64 * ceil(RW / 2), so whole 64-k steps are safe
  gemm_mainloop<SPLIT>(p.t + P.tbase[0], p.t_plane, P.RP[0], p.M, m0, P.U[0], P.RW[0], P.N, c0, (P.RW[0] + 1) / 2,
                       acc0, tid);
  if (P.nb > 1)
    gemm_mainloop<SPLIT>(p.t + P.tbase[1], p.t_plane, P.RP[1], p.M, m0, P.U[1], P.RW[1], P.N, c0,
                         (P.RW[1] + 1) / 2, acc1, tid);

  const int lane = tid & 63, wave = tid >> 6;
  const int wm = gemm_wm(wave), wn = gemm_wn(wave);
  const int lr = lane & 31, lh = lane >> 5;
  YT* __restrict__ y = static_cast<YT*>(P.y);
#pragma unroll
  for (int j = 0; j < kGNJ; ++j) {
    const int n = c0 + gemm_col<kGNJ>(wn, j) + lr;
    if (n >= P.N) continue;
    const float h0 = P.h[0][n];
    const float h1 = P.nb > 1 ? P.h[1][n] : 0.f;
    const float bn = P.bias ? P.bias[n] : 0.f;
    const float* res = P.res;
#pragma unroll
    for (int i = 0; i < kGMI; ++i)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int m = m0 + gemm_row(wm, i) + 8 * (q >> 2) + 4 * lh + (q & 3);
        if (m < p.M) {
          const size_t o = size_t(m) * P.N + n;
          store_out(y, o, h0 * acc0[i][j][q] + h1 * acc1[i][j][q] + bn + (res ? res[o] : 0.f));
        }
      }
  }
}

// Stage 2 on bf16 activations in wide tiles.  grid = (m-tiles, 256-column
// tiles of all projections), 256 threads (4 waves as in gemm_mainloop), one set of
// accumulators for both branches (two sets would not fit two blocks per CU):
// acc = S0 after branch 0 (S_b = sum_r sU_b[n, r] * T_b[m, r]), each column's
// acc times h0 / h1 in fp32, then branch 1 added: y = h1 * acc = h0 * S0 + h1
// * S1, + bias (+ residual).  Where branch 1 is dropped (use_branch1: h1
// zero, denormal or below 2^-40 |h0|, where h0 / h1 could overflow acc)
// branch 1's B operand is 0 and y = h0 * S0; the term dropped is at most
// 2^-40 of h0 times |S1 / S0|.
template <typename YT>
__global__ __launch_bounds__(kGThreads, 2) void gemm_expand_wide_kernel(GemmParams p) {
  constexpr int BN = 2 * kGB, NJ = gemm_nj<BN>();
  const int tid = int(threadIdx.x);
  const int nt = int(blockIdx.y);
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxProj; ++i) pi += (i < p.nproj && nt >= p.proj[i].nt0) ? 1 : 0;
  pi = __builtin_amdgcn_readfirstlane(pi);
  const GemmProj& P = p.proj[pi];
  const int m0 = int(blockIdx.x) * kGB;
  const int c0 = (nt - P.nt0) * BN;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = gemm_wm(wave), wn = gemm_wn(wave);
  const int lr = lane & 31, lh = lane >> 5;
  f32x16 acc[kGMI][NJ];
#pragma unroll
  for (int i = 0; i < kGMI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x16{};
  // T rows are zero from R to RP >= 64 * ceil(RW / 2), so whole 64-k steps are safe
  gemm_mainloop<false, false, BN>(p.t + P.tbase[0], p.t_plane, P.RP[0], p.M, m0, P.U[0], P.RW[0], P.N, c0,
                                  (P.RW[0] + 1) / 2, acc, tid, nullptr, 0, nullptr);
  float f[NJ];  // the factor y takes of acc, per subtile column
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = min(c0 + gemm_col<NJ>(wn, j) + lr, P.N - 1);
    const float h0 = P.h[0][n];
    const float h1 = P.nb > 1 ? P.h[1][n] : 0.f;
    const bool use1 = P.nb > 1 && use_branch1(h0, h1);
    f[j] = use1 ? h1 : h0;
    if (use1) {
      const float r = h0 / h1;
#pragma unroll
      for (int i = 0; i < kGMI; ++i) acc[i][j] *= r;
    }
  }
  if (P.nb > 1)
    gemm_mainloop<false, false, BN>(p.t + P.tbase[1], p.t_plane, P.RP[1], p.M, m0, P.U[1], P.RW[1], P.N, c0,
                                    (P.RW[1] + 1) / 2, acc, tid, nullptr, 0, P.h[1], P.h[0]);

  YT* __restrict__ y = static_cast<YT*>(P.y);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = c0 + gemm_col<NJ>(wn, j) + lr;
    if (n >= P.N) continue;
    const float bn = P.bias ? P.bias[n] : 0.f;
    const float* res = P.res;
#pragma unroll
    for (int i = 0; i < kGMI; ++i)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int m = m0 + gemm_row(wm, i) + 8 * (q >> 2) + 4 * lh + (q & 3);
        if (m < p.M) {
          const size_t o = size_t(m) * P.N + n;
          store_out(y, o, f[j] * acc[i][j][q] + bn + (res ? res[o] : 0.f));
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Sign pack / unpack (bit-exact with the reference packer)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void unpack_kernel(const uint32_t* packed, int64_t rows, int64_t cols,
                                                        int64_t wpr, int8_t* out) {
  const int64_t total = rows * cols;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < total; i += int64_t(gridDim.x) * kBlock) {
    const int64_t r = i / cols;
    const int64_t c = i - r * cols;
    const uint32_t word = packed[r * wpr + (c >> 5)];
    out[i] = int8_t(1 - 2 * int((word >> (c & 31)) & 1u));
  }
}

__global__ __launch_bounds__(kBlock) void pack_kernel(const int8_t* signs, int64_t rows, int64_t cols,
                                                      int64_t wpr, uint32_t* out) {
  const int64_t total = rows * wpr;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < total; i += int64_t(gridDim.x) * kBlock) {
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

// Sign words -> the 2-bit "i2" rows of the reference's CPU runtime
// (repack_signs_to_i2_cpu, patches/littlebit_cpu_optimized.cpp:712-764), byte
// for byte: out [rows][ob], ob = ceil(n_cols / 4).  Column c = 128 b + 32 g +
// p is the field at bits 7-6 (g = 0) .. 1-0 (g = 3) of byte 32 b + p, 2 for +1
// and 0 for -1; a column whose byte falls at or past ob is dropped and a field
// with no column stays 0.  One thread per 4 output bytes j0 .. j0 + 3 (one b,
// p .. p + 3): per g it inverts bits p .. p + 3 of word 4 b + g (+1 -> 1),
// masks the columns past n_cols and spreads the 4 bits to bit 7 - 2 g of the
// 4 bytes.  The word index 4 b + g = c / 32 of a column c < n_cols is below
// ceil(n_cols / 32) <= wpr (checked by the host).
// V sign words [R][KW] -> the latent kernel's tiled copy
// [ceil(R/16)][ceil(KW/4)][16 rows][4 words] (zero past R and past KW): a
// 16-byte cell holds 4 words of one row, and the 16 rows of a tile lie side by
// side, so the lanes of one load (16 rows x 4 word groups) read whole 128-byte
// lines whatever the k-chunk width.  One thread per cell.
__global__ __launch_bounds__(kBlock) void tile_v_kernel(const uint32_t* __restrict__ v, int64_t R, int64_t KW,
                                                        u32x4* __restrict__ out) {
  const int64_t kw4 = (KW + 3) / 4, ncell = (R + 15) / 16 * kw4 * 16;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < ncell; i += int64_t(gridDim.x) * kBlock) {
    const int64_t rl = i & 15, gi = (i >> 4) % kw4, t = (i >> 4) / kw4;
    const int64_t r = 16 * t + rl;
    u32x4 c = {0u, 0u, 0u, 0u};
    if (r < R) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (4 * gi + e < KW) c[e] = v[r * KW + 4 * gi + e];
    }
    out[i] = c;
  }
}

__global__ __launch_bounds__(kBlock) void repack_i2_kernel(const uint32_t* __restrict__ packed, int64_t rows,
                                                           int64_t wpr, int64_t n_cols, int64_t ob, int dword_rows,
                                                           uint8_t* __restrict__ out) {
  const int64_t nq = (ob + 3) / 4;
  const int64_t total = rows * nq;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < total; i += int64_t(gridDim.x) * kBlock) {
    const int64_t r = i / nq;
    const int64_t j0 = 4 * (i - r * nq);
    const int64_t b = j0 >> 5;
    const int p = int(j0 & 31);
    uint32_t d = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t c0 = 128 * b + 32 * g + p;  // column of byte j0's field g
      if (c0 < n_cols) {
        uint32_t nib = (~packed[r * wpr + 4 * b + g] >> p) & 0xfu;
        if (n_cols - c0 < 4) nib &= (1u << (n_cols - c0)) - 1u;
        const uint32_t spread = (nib & 1u) | ((nib & 2u) << 7) | ((nib & 4u) << 14) | ((nib & 8u) << 21);
        d |= spread << (7 - 2 * g);
      }
    }
    uint8_t* dst = out + r * ob + j0;
    if (dword_rows) {
      *reinterpret_cast<uint32_t*>(dst) = d;
    } else {
      const int nbytes = int(ob - j0 < 4 ? ob - j0 : 4);
      for (int e = 0; e < nbytes; ++e) dst[e] = uint8_t(d >> (8 * e));
    }
  }
}

// ---------------------------------------------------------------------------
// Decode attention: one query token per sequence, fp32, grouped KV heads,
// no rotary embedding (fused_attention_inline,
// patches/littlebit_cpu_optimized.cpp:1441-1510):
//   out[h] = sum_t softmax_t(scale * q[h] . K[h / rep][t]) V[h / rep][t],
//   t = 0 .. pos, with K/V[.][pos] = the new k, v, which are also stored in
//   the cache [kv_heads][max_seq][HD].
// grid = (heads, chunks of kAttnChunk positions), 256 threads.  A block
// scores its chunk with coalesced row reads (a group of lanes per K row,
// shuffle reduction), takes the chunk's max and exp-sum, and accumulates
// p . V with each wave on a quarter of the positions.  With one chunk it
// writes out directly, otherwise (max, sum, o[HD]) per chunk, which
// attn_combine_kernel merges.  pos is read on the device when pos_ptr is set (graph replay);
// pos >= max_seq writes nothing but zeros to out.
// ---------------------------------------------------------------------------
constexpr int kAttnThreads = 256;

struct AttnParams {
  const float* q;        // [heads * HD]
  const float* k;        // [kv_heads * HD]  new key
  const float* v;        // [kv_heads * HD]  new value
  float* kc;             // [kv_heads][max_seq][HD]
  float* vc;
  const int64_t* pos_ptr;
  int64_t pos;
  int heads, rep, max_seq, chunks;
  float scale;
  float* part;           // [heads][chunks][HD + kAttnPad]: o, max, exp-sum
  float* out;            // [heads * HD]; null: the partials are the result (a consumer merges them)
};

__device__ __forceinline__ int64_t attn_pos(const AttnParams& p) { return p.pos_ptr ? *p.pos_ptr : p.pos; }

// One wave per 16-position chunk, no barriers: grid = (heads, ceil(chunks / 4)),
// wave w of block (h, C) takes chunk 4 C + w.  K rows load LPR lanes per row
// (4 dims each), RPI rows per instruction; the NI partial dots of a lane are
// summed over its row's LPR lanes by a halving butterfly (each step sends half
// of the remaining values, so lane l ends with the full score of one row,
// held by 4 lanes); the chunk's max and exp-sum are wave reductions; p . V
// broadcasts each row's weight with v_readlane from a lane fixed at compile
// time, every lane accumulating its DPL dims over the 16 rows.
template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(AttnParams p) {
  constexpr int LPR = HD / 4, RPI = 64 / LPR, NI = kAttnChunk / RPI, DPL = HD / 64;
  constexpr int COPIES = LPR / NI;  // lanes left holding each row's score (the summing masks)
  static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
  static_assert(NI >= 2 && NI <= LPR && (NI & (NI - 1)) == 0, "rows per instruction");
  const int h = int(blockIdx.x), wave = int(threadIdx.x) >> 6, lane = int(threadIdx.x) & 63;
  const int c = int(blockIdx.y) * 4 + wave;
  const int kv = h / p.rep;
  const int64_t pos = attn_pos(p);
  if (pos < 0 || pos >= p.max_seq) {  // out of range: nothing is read or stored
    if (p.out && c == 0) {
#pragma unroll
      for (int j = 0; j < DPL; ++j) p.out[size_t(h) * HD + lane * DPL + j] = 0.f;
    }
    return;
  }
  const int S = int(pos) + 1;
  const int t0 = c * kAttnChunk;
  if (c >= p.chunks || t0 >= S) return;  // chunk past the current length: takes no part
  const float* kn = p.k + size_t(kv) * HD;
  const float* vn = p.v + size_t(kv) * HD;
  float* kc = p.kc + size_t(kv) * p.max_seq * HD;
  float* vc = p.vc + size_t(kv) * p.max_seq * HD;
  if (c == 0 && (h % p.rep) == 0) {  // store the new key / value (read below from kn, vn)
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      kc[size_t(pos) * HD + lane * DPL + j] = kn[lane * DPL + j];
      vc[size_t(pos) * HD + lane * DPL + j] = vn[lane * DPL + j];
    }
  }
  // every load first: K rows, V rows, the query (rows past the length read row t0)
  const int sub = lane / LPR, dl = (lane % LPR) * 4;
  float4 kk[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int t = t0 + i * RPI + sub;
    const float* kr = t == pos ? kn : kc + size_t(t < S ? t : t0) * HD;
    kk[i] = *reinterpret_cast<const float4*>(kr + dl);
  }
  float vv[kAttnChunk][DPL];
#pragma unroll
  for (int r = 0; r < kAttnChunk; ++r) {
    const int t = t0 + r;
    const float* vr = (t == pos ? vn : vc + size_t(t < S ? t : t0) * HD) + lane * DPL;
    if constexpr (DPL == 2) {
      const float2 w2 = *reinterpret_cast<const float2*>(vr);
      vv[r][0] = w2.x;
      vv[r][DPL - 1] = w2.y;
    } else {
      vv[r][0] = vr[0];
    }
  }
  const float4 q4 = *reinterpret_cast<const float4*>(p.q + size_t(h) * HD + dl);
  float v[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i)
    v[i] = (q4.x * kk[i].x + q4.y * kk[i].y + q4.z * kk[i].z + q4.w * kk[i].w) * p.scale;
  // halving butterfly over the LPR lanes of a row: masks LPR/2 .. 4 halve NI
  // values down to one (index bits taken from the lane), masks 2 and 1 sum
#pragma unroll
  for (int m = LPR / 2, n = NI; m >= 1; m >>= 1) {
    if (n > 1) {
      const bool up = (lane & m) != 0;
#pragma unroll
      for (int j = 0; j < NI / 2; ++j) {
        if (j < n / 2) {
          const float send = up ? v[j] : v[j + n / 2];
          const float keep = up ? v[j + n / 2] : v[j];
          v[j] = keep + __shfl_xor(send, m);
        }
      }
      n /= 2;
    } else {
      v[0] += __shfl_xor(v[0], m);
    }
  }
  // this lane's row: index bits from the halving masks, then the instruction's row
  int irow = 0;
#pragma unroll
  for (int m = LPR / 2, n = NI; n > 1; m >>= 1, n >>= 1) irow = 2 * irow + ((lane & m) ? 1 : 0);
  const int row = irow * RPI + sub;
  const float sc = t0 + row < S ? v[0] : -INFINITY;
  float mx = sc;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  const float e = t0 + row < S ? __expf(sc - mx) : 0.f;
  float sm = e * (1.0f / COPIES);  // every row is held by COPIES lanes
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) sm += __shfl_xor(sm, o);
  float o[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) o[j] = 0.f;
#pragma unroll
  for (int r = 0; r < kAttnChunk; ++r) {
    // a lane holding row r: instruction row i = r / RPI at sub r % RPI, i's
    // bits at the halving masks (the lowest, COPIES, for the lowest bit), the
    // summing-mask bits zero
    const int ir = r / RPI, sr = r % RPI;
    int ln = sr * LPR;
    int mbit = COPIES;
#pragma unroll
    for (int n = NI, k = 0; n > 1; n >>= 1, ++k, mbit <<= 1) ln |= ((ir >> k) & 1) ? mbit : 0;
    const float pr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), ln));
#pragma unroll
    for (int j = 0; j < DPL; ++j) o[j] += pr * vv[r][j];
  }
  float* part = p.part + (size_t(h) * p.chunks + c) * (HD + kAttnPad);
  if (p.chunks == 1 && p.out) {
#pragma unroll
    for (int j = 0; j < DPL; ++j) p.out[size_t(h) * HD + lane * DPL + j] = o[j] / sm;
  } else {
#pragma unroll
    for (int j = 0; j < DPL; ++j) part[lane * DPL + j] = o[j];
    if (lane == 0) {
      part[HD] = mx;
      part[HD + 1] = sm;
    }
  }
}

// out[h][d] = sum_c exp(m_c - M) o_c[d] / sum_c exp(m_c - M) l_c, M the
// largest m_c: one pass for M, one for the sums, so that every chunk's loads
// are independent (a running maximum would chain them).  grid = heads.
// sum_c exp(m_c - M) o_c[d] / sum_c exp(m_c - M) l_c over n partials
// (o[0..hd), m at hd, l at hd + 1, stride floats apart; m_c = -inf for a
// chunk that saw nothing): 16 chunks' loads at a time, rescaled online, so
// that one memory round trip covers up to 16 chunks
__device__ __forceinline__ float merge_partials(const float* __restrict__ pp, size_t stride, int n, int hd, int d) {
  float M = -INFINITY, num = 0.f, den = 0.f;
  for (int c0 = 0; c0 < n; c0 += 16) {
    float mv[16], lv[16], ov[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float* pc = pp + size_t(min(c0 + j, n - 1)) * stride;
      mv[j] = pc[hd];
      lv[j] = pc[hd + 1];
      ov[j] = pc[d];
    }
    float bm = M;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (c0 + j < n) bm = fmaxf(bm, mv[j]);
    if (bm == -INFINITY) continue;  // nothing seen yet
    const float cs = M == -INFINITY ? 0.f : __expf(M - bm);
    num *= cs;
    den *= cs;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (c0 + j < n && mv[j] != -INFINITY) {
        const float w = __expf(mv[j] - bm);
        num += w * ov[j];
        den += w * lv[j];
      }
    }
    M = bm;
  }
  return den > 0.f ? num / den : 0.f;
}

template <int HD>
__global__ __launch_bounds__(HD) void attn_combine_kernel(AttnParams p) {
  const int h = int(blockIdx.x), d = int(threadIdx.x);
  const int64_t pos = attn_pos(p);
  if (pos < 0 || pos >= p.max_seq) return;  // out was zeroed by attn_decode_kernel
  const float* part = p.part + size_t(h) * p.chunks * (HD + kAttnPad);
  const int used = int(pos / kAttnChunk) + 1;  // chunks past pos hold empty partials
  p.out[size_t(h) * HD + d] = merge_partials(part, HD + kAttnPad, used, HD, d);
}

// ---------------------------------------------------------------------------
// Attention of N new tokens (1 <= N <= 64) at positions start .. start+N-1
// over the cache and themselves, causal or with a tree mask (a new token sees
// every cached position and the new tokens its mask row marks, itself
// included when the row says so).  The reference runs its batch forward
// token by token (patches/littlebit_cpu_optimized.cpp:1846-2079) and its tree
// verification through the model's attention with the tree mask
// (tree_utils.py:72-214); here one launch covers all N tokens.
// grid = (heads, chunks of ch positions), 256 threads = 4 waves: wave w
// takes query tile w % qt (16 queries) and part w / qt of the chunk's
// positions (qt * ps = 4).  Scores S^T = K Q^T and O^T += V^T P^T run on
// v_mfma_f32_16x16x4_f32 over 16-position tiles, so products and sums stay
// fp32; the exp(scores) come out of the score MFMA in the B layout the value
// MFMA takes.  Rows at t >= start are read from the new k and v (the launch
// also stores them into the cache, for later launches).  Online softmax per
// query; the ps parts of a query tile meet in LDS, and one partial (max,
// sum, o) per (head, chunk, query) goes to attn_batch_combine_kernel.
// MFMA 16x16x4 f32 lanes: A[l % 16][l / 16], B[l / 16][l % 16], D[4 (l / 16)
// + i][l % 16].
// ---------------------------------------------------------------------------
struct AttnBatchParams {
  const float* q;         // [N][heads * HD], unscaled
  const float* k;         // [N][kv_heads * HD] new keys
  const float* v;         // [N][kv_heads * HD] new values
  float* kc;              // [kv_heads][max_seq][HD]
  float* vc;
  const uint8_t* tree;    // [N][N]: row i marks the new tokens token i sees; null: causal
  float* part;            // [heads][chunks][N][HD + 2]: o, max, sum
  float* out;             // [N][heads * HD]
  const int64_t* start_ptr;  // start read on the device when set (graph replay), else `start`
  int64_t start;
  int N, heads, kvh, rep, max_seq, chunks, ch, qt, ps;
  float scale;
};

template <int HD>
__global__ __launch_bounds__(kAttnThreads, 2) void attn_batch_kernel(AttnBatchParams p) {
  constexpr int DG = HD / 4;   // dims per lane group in the score MFMAs
  constexpr int NT = HD / 16;  // 16-dim tiles of O^T: tile 4a + b holds dims 64a + 4r + b, r < 16
  constexpr int NA = HD / 64;
  __shared__ float red[3][16][HD + 2];
  const int h = int(blockIdx.x), c = int(blockIdx.y), tid = int(threadIdx.x);
  const int wave = tid >> 6, lane = tid & 63;
  const int col = lane & 15, g = lane >> 4;
  const int kv = h / p.rep;
  const int N = p.N;
  const int64_t start = p.start_ptr ? *p.start_ptr : p.start;
  if (start < 0 || start + N > p.max_seq) return;  // out of range: nothing read or stored (the combine writes zeros)
  const int st = int(start);
  const int S = st + N;
  const int t0 = c * p.ch, t1 = min(t0 + p.ch, S);
  const size_t nstride = size_t(p.kvh) * HD;  // row stride of the new k and v
  float* kcache = p.kc + size_t(kv) * p.max_seq * HD;
  float* vcache = p.vc + size_t(kv) * p.max_seq * HD;
  const float* knew = p.k + size_t(kv) * HD;
  const float* vnew = p.v + size_t(kv) * HD;

  // the chunk's new rows into the cache (one head of each kv group stores)
  if (h % p.rep == 0) {
    const int n0 = max(t0, st), n1 = min(t1, S);
    for (int i = tid; i < (n1 - n0) * HD; i += kAttnThreads) {
      const int t = n0 + i / HD, d = i % HD;
      kcache[size_t(t) * HD + d] = knew[size_t(t - st) * nstride + d];
      vcache[size_t(t) * HD + d] = vnew[size_t(t - st) * nstride + d];
    }
  }

  const int qtile = wave % p.qt, part = wave / p.qt;
  const int qi = qtile * 16 + col;  // this lane's query: column col of the score tile
  const bool qvalid = qi < N;
  float qv[DG];
  {
    const float* qr = p.q + (size_t(min(qi, N - 1)) * p.heads + h) * HD + 4 * g;
#pragma unroll
    for (int j = 0; j < DG / 4; ++j) {
      const float4 f = *reinterpret_cast<const float4*>(qr + 16 * j);
      qv[4 * j] = f.x * p.scale;
      qv[4 * j + 1] = f.y * p.scale;
      qv[4 * j + 2] = f.z * p.scale;
      qv[4 * j + 3] = f.w * p.scale;
    }
  }
  const int P = p.ch / p.ps;
  const int w0 = t0 + part * P, w1 = min(w0 + P, t1);
  float m = -INFINITY, l = 0.f;
  f32x4 o[NT];
#pragma unroll
  for (int dt = 0; dt < NT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // K row s0 + col, dims 16 j + 4 g .. +4 for j < DG / 4 (A of the score
  // MFMAs: the 4 lanes of a row read 64 contiguous bytes per load); V rows
  // s0 + 4g + i, dims 64a + 4col .. +4 (A of the value MFMAs); positions
  // past w1 read row w1 - 1 and are masked.  The next tile's rows load while
  // this tile computes.
  auto load_kv = [&](int s0, float (&kk)[DG], float4 (&vv)[4][NA]) {
    {
      const int t = min(s0 + col, w1 - 1);
      const float* kr = (t < st ? kcache + size_t(t) * HD : knew + size_t(t - st) * nstride) + 4 * g;
#pragma unroll
      for (int j = 0; j < DG / 4; ++j) {
        const float4 f = *reinterpret_cast<const float4*>(kr + 16 * j);
        kk[4 * j] = f.x;
        kk[4 * j + 1] = f.y;
        kk[4 * j + 2] = f.z;
        kk[4 * j + 3] = f.w;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = min(s0 + 4 * g + i, w1 - 1);
      const float* vr = t < st ? vcache + size_t(t) * HD : vnew + size_t(t - st) * nstride;
#pragma unroll
      for (int a = 0; a < NA; ++a) vv[i][a] = *reinterpret_cast<const float4*>(vr + 64 * a + 4 * col);
    }
  };
  float kk[DG];
  float4 vv[4][NA];
  if (w0 < w1) load_kv(w0, kk, vv);
  for (int s0 = w0; s0 < w1; s0 += 16) {
    float kn[DG];
    float4 vn[4][NA];
    const bool more = s0 + 16 < w1;
    if (more) load_kv(s0 + 16, kn, vn);
    // four independent accumulator chains over the dims, then their sum
    f32x4 sc4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) sc4[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < DG; ++j) sc4[j % 4] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[j], qv[j], sc4[j % 4], 0, 0, 0);
    const f32x4 sc = (sc4[0] + sc4[1]) + (sc4[2] + sc4[3]);
    // sc[i] = score of position s0 + 4g + i for query qi
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = s0 + 4 * g + i;
      bool ok = qvalid && t < w1;
      if (ok && t >= st) ok = p.tree ? p.tree[size_t(qi) * N + (t - st)] != 0 : t - st <= qi;
      sv[i] = ok ? sc[i] : -INFINITY;
    }
    float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m, mx);
    const bool none = mn == -INFINITY;  // nothing visible yet: keep zeros
    const float corr = none ? 1.f : __expf(m - mn);
    float pv[4], ls = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pv[i] = none ? 0.f : __expf(sv[i] - mn);
      ls += pv[i];
    }
    ls += __shfl_xor(ls, 16);
    ls += __shfl_xor(ls, 32);
    l = l * corr + ls;
    m = mn;
#pragma unroll
    for (int dt = 0; dt < NT; ++dt) {
      o[dt] *= corr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 w = vv[i][dt / 4];
        const float a = (dt % 4) == 0 ? w.x : (dt % 4) == 1 ? w.y : (dt % 4) == 2 ? w.z : w.w;
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, pv[i], o[dt], 0, 0, 0);
      }
    }
    if (more) {
#pragma unroll
      for (int j = 0; j < DG; ++j) kk[j] = kn[j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int a = 0; a < NA; ++a) vv[i][a] = vn[i][a];
    }
  }
  // o[dt][j] = O^T[dim 64 (dt / 4) + 16 g + 4 j + dt % 4][qi]
  auto dim_of = [&](int dt, int j) { return 64 * (dt / 4) + 16 * g + 4 * j + (dt % 4); };
  if (p.ps > 1) {
    if (part > 0) {
      const int slot = qtile + p.qt * (part - 1);
#pragma unroll
      for (int dt = 0; dt < NT; ++dt)
#pragma unroll
        for (int j = 0; j < 4; ++j) red[slot][col][dim_of(dt, j)] = o[dt][j];
      if (g == 0) {
        red[slot][col][HD] = m;
        red[slot][col][HD + 1] = l;
      }
    }
    __syncthreads();
    if (part == 0) {
      for (int pi = 1; pi < p.ps; ++pi) {
        const int slot = qtile + p.qt * (pi - 1);
        const float mo = red[slot][col][HD], lo = red[slot][col][HD + 1];
        const float mn = fmaxf(m, mo);
        const float a = m == -INFINITY ? 0.f : __expf(m - mn);
        const float b = mo == -INFINITY ? 0.f : __expf(mo - mn);
        l = l * a + lo * b;
#pragma unroll
        for (int dt = 0; dt < NT; ++dt)
#pragma unroll
          for (int j = 0; j < 4; ++j) o[dt][j] = o[dt][j] * a + red[slot][col][dim_of(dt, j)] * b;
        m = mn;
      }
    }
  }
  if (part == 0 && qvalid) {
    float* pp = p.part + ((size_t(h) * p.chunks + c) * N + qi) * (HD + 2);
#pragma unroll
    for (int dt = 0; dt < NT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) pp[dim_of(dt, j)] = o[dt][j];
    if (g == 0) {
      pp[HD] = m;
      pp[HD + 1] = l;
    }
  }
}

// out[qi][h][d] = sum_c exp(m_c - M) o_c[d] / sum_c exp(m_c - M) l_c over
// the chunks' partials (merge_partials); chunks where the query sees nothing
// hold m_c = -inf.  grid = (heads, N).
template <int HD>
__global__ __launch_bounds__(HD) void attn_batch_combine_kernel(AttnBatchParams p) {
  const int h = int(blockIdx.x), qi = int(blockIdx.y), d = int(threadIdx.x);
  const int64_t start = p.start_ptr ? *p.start_ptr : p.start;
  if (start < 0 || start + p.N > p.max_seq) {
    p.out[(size_t(qi) * p.heads + h) * HD + d] = 0.f;
    return;
  }
  const size_t cstride = size_t(p.N) * (HD + 2);
  const float* pp = p.part + (size_t(h) * p.chunks * p.N + qi) * (HD + 2);
  p.out[(size_t(qi) * p.heads + h) * HD + d] = merge_partials(pp, cstride, p.chunks, HD, d);
}

// ---------------------------------------------------------------------------
// Q4_0 lm_head and argmax: the tail of the reference's generate_token
// (patches/littlebit_cpu_optimized.cpp:2254-2317).  The weight is quantised
// once to Q4_0 blocks of 32 (an fp16 scale d = m / -8 for m the block's first
// value of largest magnitude, nibbles q = min(15, int(x / d + 8.5)), value =
// (q - 8) * d; :2129-2149), stored here as two planes -- nibbles [V][H/2]
// (byte j of a block: value j low, value j + 16 high, as the reference packs
// them) and scales [V][H/32] -- so that every lane load is 16-byte aligned.
// Per call the final hidden state is (optionally RMS-normed and) quantised
// to Q8_0 (d = amax / 127, q = round(x / d); :2152-2165), each logit is
// sum_b fp16(d4_b) * fp16(d8_b) * sum_j (q4_j - 8) * q8_j (:2168-2222) and the
// token is the first index of the largest logit (:2305-2314).
// ---------------------------------------------------------------------------
constexpr int kQK = 32;  // values per Q4_0 / Q8_0 block
// rows per wave of lm_head_q4_kernel<NBL>: as many as the registers allow,
// so that the grid fits the chip in one round and fewer blocks repeat the
// Q8_0 staging
__host__ __device__ constexpr int head_rows_per_wave(int nbl) { return nbl <= 2 ? 16 : nbl == 4 ? 8 : 4; }

// fp32 -> fp16 bits as the reference converts (patch:2119-2127): exponent
// rebias, mantissa truncated, below range -> signed zero, above -> infinity
__device__ __forceinline__ uint32_t fp16_bits_trunc(float f) {
  const uint32_t v = __float_as_uint(f);
  const uint32_t sign = (v >> 16) & 0x8000u;
  const int e = int((v >> 23) & 0xFFu) - 127 + 15;
  if (e <= 0) return sign;
  if (e >= 31) return sign | 0x7C00u;
  return sign | (uint32_t(e) << 10) | ((v >> 13) & 0x3FFu);
}
__device__ __forceinline__ float fp16_value(uint32_t h) {  // exact (v_cvt_f32_f16)
  const uint16_t b = uint16_t(h);
  _Float16 v;
  __builtin_memcpy(&v, &b, sizeof(v));
  return float(v);
}

// nibble of x for scale reciprocal id: the product and the + 8.5 each
// rounded to fp32 (no fused multiply-add), then truncated
__device__ __forceinline__ uint32_t q4_nibble(float x, float id) {
#pragma clang fp contract(off)
  const float t = x * id + 8.5f;
  return uint32_t(min(15, int(t)));
}

// one thread per block of 32 weights
__global__ __launch_bounds__(256) void q4_quantize_kernel(const float* __restrict__ w, int64_t nblocks,
                                                          uint8_t* __restrict__ qs, uint16_t* __restrict__ d) {
  const int64_t b = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (b >= nblocks) return;
  const float* x = w + b * kQK;
  float v[kQK];
#pragma unroll
  for (int j = 0; j < kQK / 4; ++j) {
    const float4 f = *reinterpret_cast<const float4*>(x + 4 * j);
    v[4 * j] = f.x;
    v[4 * j + 1] = f.y;
    v[4 * j + 2] = f.z;
    v[4 * j + 3] = f.w;
  }
  float amax = 0.f, m = 0.f;
#pragma unroll
  for (int j = 0; j < kQK; ++j)
    if (fabsf(v[j]) > amax) {  // strictly greater: the first of equal magnitudes
      amax = fabsf(v[j]);
      m = v[j];
    }
  const float dv = m / -8.0f;
  const float id = dv != 0.f ? 1.0f / dv : 0.f;
  uint32_t words[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t wd = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = 4 * k + e;
      wd |= (q4_nibble(v[j], id) | (q4_nibble(v[j + 16], id) << 4)) << (8 * e);
    }
    words[k] = wd;
  }
  *reinterpret_cast<uint4*>(qs + b * 16) = uint4{words[0], words[1], words[2], words[3]};
  d[b] = uint16_t(fp16_bits_trunc(dv));
}

struct Q4HeadParams {
  const uint8_t* qs;   // [V][H/2]
  const uint16_t* d;   // [V][H/32] fp16 bits
  const float* x;      // [H] final hidden (before the norm when nw is set)
  const float* nw;     // [H] final RMSNorm weight, or null
  float eps;
  int V, H;
  float* logits;       // [V] or null
  uint64_t* part;      // [gridDim.x] (value, index) keys of each block's best
  int64_t* token;      // argmax
  int nparts;
};

// larger key = larger logit, then smaller index (the first maximum wins)
__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (uint64_t(o) << 32) | uint64_t(0xFFFFFFFFu - uint32_t(idx));
}

// grid = blocks of 4 waves, head_rows_per_wave(NBL) rows per wave.  Every block first
// builds the Q8_0 copy of the hidden state in LDS, a thread per block of 32
// (x, and the norm weight, 16-byte aligned; RMSNorm applied as
// rms_norm_inline does: x * (1 / sqrt(sum x^2 / H + eps)) * w; patch:1370-1405),
// while lane l's loads of blocks l, l + 64, .. of each of the wave's rows
// (one 16-byte nibble load and one scale per block, issued first) are in
// flight; the dot
// products on v_dot4_i32_i8 (nibbles 0..15 as signed bytes, minus 8 * sum q8).
template <int NBL>
__global__ __launch_bounds__(256) void lm_head_q4_kernel(Q4HeadParams p) {
  constexpr int HMAX = NBL * 64 * kQK;
  constexpr int kHeadRowsPerWave = head_rows_per_wave(NBL);
  __shared__ uint32_t q8w[HMAX / 4];
  __shared__ float d8[HMAX / kQK];
  __shared__ int s8[HMAX / kQK];
  __shared__ float red[4];
  __shared__ uint64_t best[4];
  const int tid = int(threadIdx.x), wave = tid >> 6, lane = tid & 63;
  const int H = p.H, nb = H / kQK;
  // the wave's rows first: their latency overlaps the staging below
  const int r0 = (int(blockIdx.x) * 4 + wave) * kHeadRowsPerWave;
  uint4 wq[kHeadRowsPerWave][NBL];
  uint32_t wd[kHeadRowsPerWave][NBL];
#pragma unroll
  for (int rr = 0; rr < kHeadRowsPerWave; ++rr) {
    const int r = min(r0 + rr, p.V - 1);
#pragma unroll
    for (int i = 0; i < NBL; ++i) {
      const int b = min(lane + 64 * i, nb - 1);
      wq[rr][i] = *reinterpret_cast<const uint4*>(p.qs + size_t(r) * (H / 2) + size_t(b) * 16);
      wd[rr][i] = p.d[size_t(r) * nb + b];
    }
  }
  // Q8_0 of the hidden state: thread t quantises blocks t, t + 256, .. from
  // its own registers (no cross-lane steps); the RMSNorm's sum of squares is
  // the one block-wide reduction
  constexpr int BPT = (HMAX / kQK + 255) / 256;  // Q8 blocks per thread
  float xv[BPT][kQK], wv[BPT][kQK];
#pragma unroll
  for (int c = 0; c < BPT; ++c) {
    const int b = min(tid + 256 * c, nb - 1);
#pragma unroll
    for (int q = 0; q < kQK / 4; ++q) {
      const float4 f = *reinterpret_cast<const float4*>(p.x + b * kQK + 4 * q);
      xv[c][4 * q] = f.x;
      xv[c][4 * q + 1] = f.y;
      xv[c][4 * q + 2] = f.z;
      xv[c][4 * q + 3] = f.w;
      if (p.nw) {
        const float4 g = *reinterpret_cast<const float4*>(p.nw + b * kQK + 4 * q);
        wv[c][4 * q] = g.x;
        wv[c][4 * q + 1] = g.y;
        wv[c][4 * q + 2] = g.z;
        wv[c][4 * q + 3] = g.w;
      }
    }
  }
  float rs = 1.f;
  if (p.nw) {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < BPT; ++c)
      if (tid + 256 * c < nb) {
#pragma unroll
        for (int j = 0; j < kQK; ++j) ss += xv[c][j] * xv[c][j];
      }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    rs = 1.0f / sqrtf(ss / float(H) + p.eps);
  }
#pragma unroll
  for (int c = 0; c < BPT; ++c) {
    const int b = tid + 256 * c;
    if (b >= nb) break;
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < kQK; ++j) {
      if (p.nw) xv[c][j] = xv[c][j] * rs * wv[c][j];
      amax = fmaxf(amax, fabsf(xv[c][j]));
    }
    const float dv = amax / 127.0f;
    const float id = dv != 0.f ? 1.0f / dv : 0.f;
    uint32_t qw[kQK / 4];
    int sq = 0;
#pragma unroll
    for (int q = 0; q < kQK / 4; ++q) {
      uint32_t wd4 = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int v = int(roundf(xv[c][4 * q + e] * id));
        sq += v;
        wd4 |= (uint32_t(v) & 0xFFu) << (8 * e);
      }
      qw[q] = wd4;
    }
    uint4* dst = reinterpret_cast<uint4*>(q8w + b * 8);
    dst[0] = uint4{qw[0], qw[1], qw[2], qw[3]};
    dst[1] = uint4{qw[4], qw[5], qw[6], qw[7]};
    d8[b] = fp16_value(fp16_bits_trunc(dv));
    s8[b] = sq;
  }
  __syncthreads();
  // this lane's blocks of the activation, for every row
  uint32_t qa[NBL][8];
  float da[NBL];
  int sa[NBL];
#pragma unroll
  for (int i = 0; i < NBL; ++i) {
    const int b = min(lane + 64 * i, nb - 1);
#pragma unroll
    for (int k = 0; k < 8; ++k) qa[i][k] = q8w[b * 8 + k];
    da[i] = lane + 64 * i < nb ? d8[b] : 0.f;  // lanes past the row add nothing
    sa[i] = s8[b];
  }
  uint64_t mine = 0;
#pragma unroll
  for (int rr = 0; rr < kHeadRowsPerWave; ++rr) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NBL; ++i) {
      const uint32_t w4[4] = {wq[rr][i].x, wq[rr][i].y, wq[rr][i].z, wq[rr][i].w};
      int sumi = -8 * sa[i];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        sumi = __builtin_amdgcn_sdot4(int(w4[k] & 0x0F0F0F0Fu), int(qa[i][k]), sumi, false);
        sumi = __builtin_amdgcn_sdot4(int((w4[k] >> 4) & 0x0F0F0F0Fu), int(qa[i][4 + k]), sumi, false);
      }
      acc += (fp16_value(wd[rr][i]) * da[i]) * float(sumi);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
    const int r = r0 + rr;
    if (r < p.V) {
      if (p.logits && lane == 0) p.logits[r] = acc;
      const uint64_t k = argmax_key(acc, r);
      mine = k > mine ? k : mine;
    }
  }
  if (lane == 0) best[wave] = mine;
  __syncthreads();
  if (tid == 0) {
    uint64_t m = best[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) m = best[w] > m ? best[w] : m;
    p.part[blockIdx.x] = m;
  }
}

// one block: the largest key of the blocks' bests -> token
__global__ __launch_bounds__(256) void argmax_finalize_kernel(Q4HeadParams p) {
  __shared__ uint64_t red[4];
  const int tid = int(threadIdx.x);
  uint64_t m = 0;
  for (int base = 0; base < p.nparts; base += 256 * 8) {  // eight loads in flight per round
    uint64_t v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = base + tid + 256 * k;
      v[k] = i < p.nparts ? p.part[i] : 0;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) m = v[k] > m ? v[k] : m;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint64_t other = __shfl_xor(m, o);
    m = other > m ? other : m;
  }
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) m = red[w] > m ? red[w] : m;
    m = red[0] > m ? red[0] : m;
    *p.token = int64_t(0xFFFFFFFFu - uint32_t(m & 0xFFFFFFFFu));
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(LBK_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return LBK_OK;
}

// One projection of a group call as the host sees it.
struct ProjDesc {
  const lbk_branch* br;
  int nb;
  int64_t N;
  const float* bias;
  void* y;
  const float* res;
};

// The call's effective input (LBK_INPUT_*).
struct InputDesc {
  int kind;
  const float* nw;
  float eps;
  const void* x1;
  int head_dim, max_seq;      // LBK_INPUT_ATTN_MERGE
  const int64_t* pos_device;
  int64_t pos;
};

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; }

int validate_group(const ProjDesc* pd, int np, int64_t M, int64_t K) {
  if (np < 1 || np > kMaxProj) return set_error(LBK_ERR_ARG, "n_proj must be in [1, %d], got %d", kMaxProj, np);
  if (M < 0 || M > kMaxDim)
    return set_error(LBK_ERR_ARG, "M must be in [0, %lld], got %lld", (long long)kMaxDim, (long long)M);
  if (K < 1 || K > kMaxDim)
    return set_error(LBK_ERR_ARG, "K must be in [1, %lld], got %lld", (long long)kMaxDim, (long long)K);
  int64_t rsum = 0;
  for (int q = 0; q < np; ++q) {
    const ProjDesc& P = pd[q];
    if (!P.br) return set_error(LBK_ERR_ARG, "projection %d: branches is NULL", q);
    if (P.nb < 1 || P.nb > 2)
      return set_error(LBK_ERR_ARG, "projection %d: n_branches must be 1 or 2, got %d", q, P.nb);
    if (P.N < 1 || P.N > kMaxDim)
      return set_error(LBK_ERR_ARG, "projection %d: N must be in [1, %lld], got %lld", q, (long long)kMaxDim,
                       (long long)P.N);
    for (int b = 0; b < P.nb; ++b) {
      const lbk_branch& B = P.br[b];
      if (B.rank < 1)
        return set_error(LBK_ERR_ARG, "projection %d branch %d: rank must be >= 1, got %lld", q, b,
                         (long long)B.rank);
      if (!B.v_sign || !B.u_sign || !B.v2 || !B.mid || !B.u1)
        return set_error(LBK_ERR_ARG, "projection %d branch %d: NULL factor or scale pointer", q, b);
      if (B.v_sign_tiled && (reinterpret_cast<uintptr_t>(B.v_sign_tiled) & 15u))
        return set_error(LBK_ERR_ARG, "projection %d branch %d: v_sign_tiled must be 16-byte aligned", q, b);
      rsum += B.rank;
    }
  }
  if (rsum > kMaxRankTotal)
    return set_error(LBK_ERR_ARG, "sum of branch ranks %lld exceeds %lld", (long long)rsum, (long long)kMaxRankTotal);
  return LBK_OK;
}

// Workspace layout (byte offsets), fixed so that calls of any shape on one
// workspace keep its invariants:
//   [0, 16)                            latent-buffer state (see MfmaParams)
//   [kSkCntOffset, + 4 kSkMaxBlocks)   stream-K step counters (zero between calls)
//   [kDetCntOffset, + 4 kDetMaxBlocks) deterministic mode's row-block counters (zero
//                                      between calls)
//   [kTOffset, kTOffset + kTBytes)     MFMA-path latent halves
//   [kChainOffset, + kChainBytes)      chains' latent regions (zero between
//                                      chains but for the last region)
//   [kGemmOffset, ...)                 one call's own scratch: GEMM-path A and
//                                      T planes, then the stream-K partial
//                                      tiles (kSkPartBytes); or deterministic
//                                      mode's partial sums
constexpr size_t kTOffset = 4096;
constexpr size_t kTBytes = 2 * size_t(kTHalf) * sizeof(float);
constexpr size_t kChainOffset = kTOffset + kTBytes;
constexpr size_t kChainBytes = size_t(kMaxChainLinks) * kChainRegion * sizeof(float);
constexpr size_t kGemmOffset = kChainOffset + kChainBytes;
static_assert(kCounterBytes <= kTOffset, "counter region overlaps t");
constexpr int kNumCUs = 256;                   // MI355X
constexpr int kSkMaxBlocks = 2 * kNumCUs;      // stream-K blocks: two resident per CU (bf16 stage ring)
constexpr size_t kSkCntOffset = 256;
static_assert(kSkCntOffset + kSkMaxBlocks * sizeof(uint32_t) <= kCounterBytes, "stream-K counters");
constexpr int kDetMaxBlocks = int(kMaxRankTotal / kRowBlock) + kMaxSeg;  // row-blocks of one decode-path call
constexpr size_t kDetCntOffset = kSkCntOffset + kSkMaxBlocks * sizeof(uint32_t);
static_assert(kDetCntOffset + kDetMaxBlocks * sizeof(uint32_t) <= kCounterBytes, "deterministic-mode counters");
constexpr size_t kSkSlotBytes = size_t(64) * kGThreads * sizeof(float);  // one fp32 partial tile

// Stream-K blocks of stage 1, or 0 when whole tiles do as well.  Costs in
// k-steps of one block alone on a CU, as measured on the config-4 shapes at
// M = 128 .. 2048: two co-resident blocks each take 1.5x as long per step,
// and a stream-K block pays about 24 steps more (its extra ring prologues
// and the partial tiles).  Whole tiles: nks when each CU gets at most one,
// else ceil(tiles / 2 CUs) rounds of 1.5 nks.  P stream-K blocks: W / P + 24,
// times 1.5 when P > CUs.  P is at most the resident slots, about 4 steps
// per block and 4 parts per tile (the part that completes a tile reads the
// others' 64 KB partial tiles on its own); the better of P <= CUs and P <=
// slots, and only if it saves 5 %.
int64_t sk_blocks(int64_t tiles, int64_t nks, int slots) {
  if (tiles < 1 || nks < 1) return 0;  // M = 0: nothing to share
  const int64_t work = tiles * nks, cap = std::min<int64_t>(std::max<int64_t>(1, work / 4), 4 * tiles);
  // costs doubled, to keep the factor 1.5 in integers
  const int64_t dp = tiles <= kNumCUs ? 2 * nks : ceil_div(tiles, int64_t(2 * kNumCUs)) * 3 * nks;
  int64_t best = 0, best_cost = dp * 95 / 100;
  for (int64_t lim : {int64_t(kNumCUs), int64_t(slots)}) {
    const int64_t P = std::min(lim, cap);
    const int64_t cost = (P > kNumCUs ? 3 : 2) * (ceil_div(work, P) + 24);
    if (cost < best_cost) {
      best = P;
      best_cost = cost;
    }
  }
  return best;
}

// Column tiles of stage 1 over all branches.
int64_t latent_col_tiles(const ProjDesc* pd, int np) {
  int64_t nt = 0;
  for (int q = 0; q < np; ++q)
    for (int b = 0; b < pd[q].nb; ++b) nt += ceil_div(pd[q].br[b].rank, kGB);
  return nt;
}

// Deterministic mode (lbk_set_deterministic): process-wide; read when a
// call is planned, so a workspace sized while it was off may be too small
// for a call made after it is turned on (that call returns
// LBK_ERR_WORKSPACE).
std::atomic<int> g_deterministic{0};

// Floats of the deterministic partials of a decode-path call: nkc copies of t
// (M * sum of 32 * RWp per branch) and 2 * nkc sub-slots of kMaxMfmaM sums
// of squares.
size_t det_part_floats(const ProjDesc* pd, int np, int64_t M, int nkc) {
  int64_t tsize = 0;
  for (int q = 0; q < np; ++q)
    for (int b = 0; b < pd[q].nb; ++b) tsize += M * 32 * ceil_div(ceil_div(pd[q].br[b].rank, 32), 4) * 4;
  return size_t(nkc) * size_t(tsize) + size_t(2 * nkc) * kMaxMfmaM;
}

// Launch plan shared by the workspace query and the forward.
struct Plan {
  bool mfma;
  int mt;        // M tile of the MFMA path: 1, 2, 4, 8 or 16
  int wpl;       // words per lane in latent_mfma_kernel
  int nkc;       // k-chunks
  int nrb;       // row-blocks over all segments
  int wsteps;    // expand_mfma_kernel unroll bound S
  int waves;     // expand_mfma_kernel waves per block (4, 8 or 12)
  int splits;    // expand_mfma_kernel waves per 16-row tile
  int ks;        // expand_mfma_kernel rank slices (grid.y)
  bool allow_ks; // rank slices were allowed (chunks plan with the same rule)
  int chunk;     // > 0: rows per decode-path call, the call runs over chunks of rows
  bool det;      // deterministic mode, read once when the call is planned
  bool seq;      // chunk > 0: one launch pair per chunk, one chunk after another
  bool reverse;  // seq: the chunks run last to first (an output overlapping the input)
  size_t lds1, lds2;
  size_t ws_total;  // workspace the fastest form of the call uses
  size_t ws_min;    // workspace it needs (GEMM path: without the stream-K partial tiles)
};

int mtile(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// 16-byte rows of a compact operand with `nch` chunks
size_t compact_rows(int mt, int64_t nch) {
  const int mb = (mt + 7) / 8, mr = mt < 8 ? mt : 8;
  return size_t(mb) * size_t(nch) * size_t(2 * mr + 1);
}


// Elements per plane of the GEMM path's A (per segment [M][Kp]) and T (per
// segment [M][RP]); planes are bf16, two of each with SPLIT.
void gemm_planes(const ProjDesc* pd, int np, int64_t M, int64_t K, int64_t& a_plane, int64_t& t_plane) {
  a_plane = t_plane = 0;
  const int64_t Kp = ceil_div(K, kGK) * kGK;
  for (int q = 0; q < np; ++q)
    for (int b = 0; b < pd[q].nb; ++b) {
      a_plane += M * Kp;
      t_plane += M * ceil_div(pd[q].br[b].rank, kGB) * kGB;
    }
}

size_t gemm_ws_bytes(const ProjDesc* pd, int np, int64_t M, int64_t K, bool split) {
  int64_t ap, tp;
  gemm_planes(pd, np, M, K, ap, tp);
  const size_t planes = split ? 2 : 1;
  return align256(size_t(ap) * planes * sizeof(uint16_t)) + align256(size_t(tp) * planes * sizeof(uint16_t));
}

// Static LDS of expand_mfma_kernel (the `red` array).
size_t expand_static_lds(int waves, int mt) { return size_t(waves) * ((mt + 7) / 8) * 4 * 32 * sizeof(float); }

struct ExpandChoice {
  int waves = 0, splits = 0, ws = 0, ks = 1;  // waves 0: no shape fits
  size_t lds2 = 0;                            // dynamic LDS (the slice's t chunks)
};

// Expand launch shape: waves per block (4, 8 or 12), waves per 16-row tile
// (splits) and rank slices (ks), by an estimate of the kernel's critical path
// in half rank steps of one wave: the t staging weighs a round trip to L2 (8
// steps) plus 2 steps per 32-byte row load each thread issues (chunks x rows
// / threads), and repeats for each round of blocks the CUs cannot hold at
// once (blocks per CU bounded by LDS, by 2048 threads and by the kernel's
// registers); the busiest SIMD then runs ceil(blocks / 256) * waves / 4 waves
// of part_steps() steps each, weighted 1.5.  Ties go to fewer blocks (less
// staging traffic).  The weights were fitted to a sweep of every (waves,
// splits, ks) over the Llama-2 draft and target calls at M = 1, 8, 16 and
// 33 on MI355X (32 calls: the picks' total 500.6 -> 493.8 us against 479.5
// for the best shape of each call; no M = 1 draft pick changed).
// Rank steps of projection q as expand_mfma_kernel walks them (branch 0's
// padded to a multiple of 4 when branch 1 follows) and the steps of one of
// `splits` parts.
int64_t proj_steps(const ProjDesc& d) {
  const int64_t st0 = ceil_div(ceil_div(d.br[0].rank, 32), 4);
  return d.nb > 1 ? (st0 + 3) / 4 * 4 + ceil_div(ceil_div(d.br[1].rank, 32), 4) : st0;
}
// Slice s of ks: groups of 4 steps [s * ng / ks, (s + 1) * ng / ks) (as in
// expand_mfma_kernel); its steps [a, b) and the t chunks it stages (16 per
// step of either branch; branch 0's padding steps have none).
void slice_range(const ProjDesc& d, int ks, int s, int64_t& a, int64_t& b) {
  const int64_t n = proj_steps(d), ng = ceil_div(n, 4);
  a = std::min(n, 4 * (s * ng / ks));
  b = std::min(n, 4 * ((s + 1) * ng / ks));
}
int64_t slice_chunks(const ProjDesc& d, int ks, int s) {
  int64_t a, b;
  slice_range(d, ks, s, a, b);
  const int64_t st0 = ceil_div(ceil_div(d.br[0].rank, 32), 4);
  int64_t steps = std::max<int64_t>(0, std::min(b, st0) - a);
  if (d.nb > 1) {
    const int64_t p0 = (st0 + 3) / 4 * 4;
    steps += std::max<int64_t>(0, b - std::max(a, p0));
  }
  return 16 * steps;
}
// Steps of one of `splits` parts of the longest slice.
int64_t part_steps(const ProjDesc& d, int splits, int ks) {
  int64_t n = 0;
  for (int s = 0; s < ks; ++s) {
    int64_t a, b;
    slice_range(d, ks, s, a, b);
    n = std::max(n, b - a);
  }
  return d.nb > 1 ? 4 * ceil_div(n, 4 * splits) : ceil_div(n, splits);
}

// Wave-step bucket (the S of expand_mfma_kernel) of a wave's ws steps.
int wave_step_bucket(int64_t ws) { return ws <= 4 ? 4 : ws <= 8 ? 8 : ws <= 16 ? 16 : ws <= 24 ? 24 : kMaxWaveSteps; }

// Blocks of expand_mfma_kernel<float, MT, S, WAVES> that one CU holds by its
// registers and wave slots: the runtime's occupancy query without dynamic
// LDS (the caller bounds LDS itself), once per instantiation.  0 where the
// query fails (no device): the caller then counts LDS and threads only.
template <int MT, int S, int WAVES>
int expand_occupancy_one() {
  static std::atomic<int> cached{-1};
  int v = cached.load(std::memory_order_relaxed);
  if (v < 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(&expand_mfma_kernel<float, MT, S, WAVES>), WAVES * kWave, 0) !=
        hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    v = std::max(n, 0);
    cached.store(v, std::memory_order_relaxed);
  }
  return v;
}
template <int MT, int S>
int expand_occupancy_w(int waves) {
  if constexpr (MT <= 8) {
    if (waves == 12) return expand_occupancy_one<MT, S, 12>();
  }
  return waves == 8 ? expand_occupancy_one<MT, S, 8>() : expand_occupancy_one<MT, S, 4>();
}
template <int MT>
int expand_occupancy_s(int64_t ws, int waves) {
  switch (wave_step_bucket(ws)) {
    case 4: return expand_occupancy_w<MT, 4>(waves);
    case 8: return expand_occupancy_w<MT, 8>(waves);
    case 16: return expand_occupancy_w<MT, 16>(waves);
    case 24: return expand_occupancy_w<MT, 24>(waves);
    default: return expand_occupancy_w<MT, kMaxWaveSteps>(waves);
  }
}
int expand_occupancy(int mt, int64_t ws, int waves) {
  switch (mt) {
    case 1: return expand_occupancy_s<1>(ws, waves);
    case 2: return expand_occupancy_s<2>(ws, waves);
    case 4: return expand_occupancy_s<4>(ws, waves);
    case 8: return expand_occupancy_s<8>(ws, waves);
    default: return expand_occupancy_s<16>(ws, waves);
  }
}

ExpandChoice expand_shape(const ProjDesc* pd, int np, int mt, bool allow_ks, int nchunks) {
  constexpr int kCUs = 256;
  ExpandChoice best;
  int64_t best_key[2] = {INT64_MAX, INT64_MAX};
  const int64_t mb = (mt + 7) / 8;
  int64_t ng_min = INT64_MAX;  // groups of 4 steps of the shortest sequence
  for (int q = 0; q < np; ++q) ng_min = std::min(ng_min, ceil_div(proj_steps(pd[q]), 4));
  for (int ks : {1, 2, 3, 4, 6, 8}) {
    if (ks > 1 && (!allow_ks || ks > ng_min)) break;
    // the largest slice's t chunks over the projections
    int64_t chunks = 0;
    for (int q = 0; q < np; ++q)
      for (int s = 0; s < ks; ++s) chunks = std::max(chunks, slice_chunks(pd[q], ks, s));
    const size_t lds2 = compact_rows(mt, chunks) * 16;
    for (int waves : {4, 8, 12}) {
      if (waves == 12 && mt > 8) continue;  // 12 waves of the M = 16 kernel spill
      const int threads = waves * kWave;
      const size_t lds = lds2 + expand_static_lds(waves, mt);
      if (lds > size_t(kMaxBlockLds)) continue;
      for (int splits = 1; splits <= waves; splits *= 2) {
        if (waves % splits) continue;
        int64_t ws = 0;
        for (int q = 0; q < np; ++q) ws = std::max(ws, part_steps(pd[q], splits, ks));
        if (ws > kMaxWaveSteps) continue;
        const int occ = expand_occupancy(mt, ws, waves);
        const int64_t per_cu = std::max<int64_t>(
            1, std::min<int64_t>({int64_t(kLdsPerCU) / int64_t(lds), 2048 / threads, occ > 0 ? occ : INT64_MAX}));
        const int tiles = waves / splits;
        int64_t blocks = 0;
        for (int q = 0; q < np; ++q) blocks += ceil_div(pd[q].N, 16 * tiles) * ks * nchunks;
        const int64_t rounds = ceil_div(blocks, kCUs * per_cu);
        const int64_t stage = rounds * (8 + 2 * ceil_div(chunks * mt, threads));
        const int64_t cost = 2 * stage + 3 * ceil_div(blocks, kCUs) * (waves / 4) * ws * mb;
        const int64_t key[2] = {cost, blocks};
        if (std::lexicographical_compare(key, key + 2, best_key, best_key + 2)) {
          best.waves = waves;
          best.splits = splits;
          best.ws = int(ws);
          best.ks = ks;
          best.lds2 = lds2;
          std::copy(key, key + 2, best_key);
        }
      }
    }
  }
  return best;
}

// allow_ks: the expand stage may cut the rank into slices that add their
// parts to y with fp32 atomics (fp32 y, not overlapping the inputs, and not
// in deterministic mode).
// nchunks: row chunks of this plan's rows that run side by side in one
// launch pair (the expand kernel's blocks multiply by it).
Plan plan_one(const ProjDesc* pd, int np, int64_t M, int64_t K, bool allow_ks, bool det, int nchunks = 1) {
  Plan pl{};
  pl.allow_ks = allow_ks;
  pl.det = det;
  int64_t nrb = 0;
  pl.mt = mtile(M);
  bool small_u = false;  // a U matrix of fewer than 4 words: no 16-byte sign loads
  for (int q = 0; q < np; ++q) {
    for (int b = 0; b < pd[q].nb; ++b) {
      const int64_t R = pd[q].br[b].rank;
      small_u = small_u || pd[q].N * ceil_div(R, 32) < 4;
      nrb += ceil_div(R, kRowBlock);
    }
  }
  pl.nrb = int(nrb);
  // no rank slices for one row: the kernels then fold the slice arithmetic
  // away (draft step 1.183 -> 1.163 ms; the target's one-row calls 50.8 ->
  // 49.6 us per layer with the one-row chunk folding)
  const ExpandChoice ex = expand_shape(pd, np, pl.mt, allow_ks && pl.mt > 1, nchunks);
  pl.mfma = M >= 1 && M <= kMaxMfmaM && ex.waves > 0 && !small_u;
  if (pl.mfma) {
    // the widest k-chunks that still give 384 blocks over all row chunks
    // side by side (1.5 per CU: measured 1-1.6 us faster per layer's calls
    // than 256 at 1-33 rows of the target's gate/up and o, the draft's picks
    // at one row unchanged), short per-wave chains (MT * WPL <= 64 keeps the
    // staging at <= 4 rows per thread)
    pl.wpl = 2;
    for (int w : {8, 4}) {
      if (pl.mt * w <= 64 && nrb * ceil_div(K, 128 * w) * nchunks >= 384) { pl.wpl = w; break; }
    }
    pl.nkc = int(ceil_div(K, 128 * pl.wpl));
    pl.wsteps = wave_step_bucket(ex.ws);
    pl.lds1 = compact_rows(pl.mt, 128 * pl.wpl / 8) * 16;
    pl.lds2 = ex.lds2;
    pl.waves = ex.waves;
    pl.splits = ex.splits;
    pl.ks = ex.ks;
    pl.ws_total = pl.ws_min = kTOffset + kTBytes;
    if (det && pl.nkc > 1)
      pl.ws_total = pl.ws_min = kGemmOffset + align256(det_part_floats(pd, np, M, pl.nkc) * sizeof(float));
  } else {
    pl.ws_min = kGemmOffset + gemm_ws_bytes(pd, np, M, K, true);
    const int64_t tiles = ceil_div(M, kGB) * latent_col_tiles(pd, np), nks = ceil_div(K, kGK);
    const int64_t P = std::max(sk_blocks(tiles, nks, 2 * kNumCUs), sk_blocks(tiles, nks, kNumCUs));
    pl.ws_total = pl.ws_min + size_t(2 * P) * kSkSlotBytes;
  }
  return pl;
}

// A few rows more than the decode path takes at once (or rows whose t does
// not fit in LDS) run as decode-path calls over chunks of rows: the GEMM
// path's 128-row tiles leave a handful of blocks per call at such M (e.g. 17
// blocks for the latent stage of a Llama-2 o projection at M = 33).  Rows of
// a call are independent, so the chunks compute what one call would.
constexpr int64_t kMaxChunkedM = 64;

// Whether M rows of the projections' latent vectors and their sums of
// squares fit one latent half.
bool t_fits(const ProjDesc* pd, int np, int64_t M) {
  int64_t rp = 0;
  for (int q = 0; q < np; ++q)
    for (int b = 0; b < pd[q].nb; ++b) rp += 32 * ceil_div(ceil_div(pd[q].br[b].rank, 32), 4) * 4;
  return M <= kSsqSlots && M * rp + kSsqSlots <= kTHalf;
}

// Chunk rows: 8 where the chunks run side by side (more, lighter blocks:
// measured 16 % faster than 16-row chunks at 17-40 rows of the Llama-2 target
// calls), else 16 (one launch pair per chunk: fewer pairs).  Side by side,
// 9-16 rows also go as 8-row chunks rather than one 16-row pass (measured 6-11
// % faster at 9, 12 and 16 rows over the draft and target calls).
Plan make_plan(const ProjDesc* pd, int np, int64_t M, int64_t K, bool allow_ks, bool det) {
  const Plan pl = plan_one(pd, np, M, K, allow_ks, det);
  const bool side_by_side = !det && t_fits(pd, np, M);
  if ((!pl.mfma || (M > 8 && side_by_side)) && M > 1 && M <= kMaxChunkedM) {
    for (int64_t c : {side_by_side ? int64_t(8) : int64_t(16), side_by_side ? int64_t(16) : int64_t(8)}) {
      if (c >= M) continue;
      Plan pc = plan_one(pd, np, c, K, allow_ks, det, side_by_side ? int(ceil_div(M, c)) : 1);
      if (pc.mfma) {
        pc.chunk = int(c);
        pc.seq = !side_by_side;
        return pc;
      }
    }
  }
  return pl;
}

template <typename XT, int MT, int WPL>
void launch_latent_mfma(const MfmaParams& p, dim3 grid, size_t lds, hipStream_t s) {
  if (p.part) hipLaunchKernelGGL((latent_mfma_kernel<XT, MT, WPL, true>), grid, dim3(kBlock), lds, s, p);
  else hipLaunchKernelGGL((latent_mfma_kernel<XT, MT, WPL, false>), grid, dim3(kBlock), lds, s, p);
}

template <typename XT, int MT>
void dispatch_latent_wpl(const MfmaParams& p, int wpl, dim3 grid, size_t lds, hipStream_t s) {
  switch (wpl) {
    case 8: launch_latent_mfma<XT, MT, 8>(p, grid, lds, s); break;
    case 4: launch_latent_mfma<XT, MT, 4>(p, grid, lds, s); break;
    default: launch_latent_mfma<XT, MT, 2>(p, grid, lds, s); break;
  }
}

template <typename XT>
void dispatch_latent(const MfmaParams& p, const Plan& pl, dim3 grid, hipStream_t s) {
  switch (pl.mt) {
    case 1: dispatch_latent_wpl<XT, 1>(p, pl.wpl, grid, pl.lds1, s); break;
    case 2: dispatch_latent_wpl<XT, 2>(p, pl.wpl, grid, pl.lds1, s); break;
    case 4: dispatch_latent_wpl<XT, 4>(p, pl.wpl, grid, pl.lds1, s); break;
    case 8: dispatch_latent_wpl<XT, 8>(p, pl.wpl, grid, pl.lds1, s); break;
    default: dispatch_latent_wpl<XT, 16>(p, pl.wpl, grid, pl.lds1, s); break;
  }
}

template <typename YT, int MT, int S, int WAVES>
void launch_expand_mfma(const MfmaParams& p, dim3 grid, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((expand_mfma_kernel<YT, MT, S, WAVES>), grid, dim3(WAVES * kWave), lds, s, p);
}

template <typename YT, int MT, int S>
void dispatch_expand_waves(const MfmaParams& p, int waves, dim3 grid, size_t lds, hipStream_t s) {
  if constexpr (MT <= 8) {
    if (waves == 12) {
      launch_expand_mfma<YT, MT, S, 12>(p, grid, lds, s);
      return;
    }
  }
  if (waves == 8) launch_expand_mfma<YT, MT, S, 8>(p, grid, lds, s);
  else launch_expand_mfma<YT, MT, S, 4>(p, grid, lds, s);
}

template <typename YT, int MT>
void dispatch_expand_s(const MfmaParams& p, const Plan& pl, dim3 grid, hipStream_t s) {
  switch (pl.wsteps) {
    case 4: dispatch_expand_waves<YT, MT, 4>(p, pl.waves, grid, pl.lds2, s); break;
    case 8: dispatch_expand_waves<YT, MT, 8>(p, pl.waves, grid, pl.lds2, s); break;
    case 16: dispatch_expand_waves<YT, MT, 16>(p, pl.waves, grid, pl.lds2, s); break;
    case 24: dispatch_expand_waves<YT, MT, 24>(p, pl.waves, grid, pl.lds2, s); break;
    default: dispatch_expand_waves<YT, MT, kMaxWaveSteps>(p, pl.waves, grid, pl.lds2, s); break;
  }
}

template <typename YT>
void dispatch_expand(const MfmaParams& p, const Plan& pl, dim3 grid, hipStream_t s) {
  switch (pl.mt) {
    case 1: dispatch_expand_s<YT, 1>(p, pl, grid, s); break;
    case 2: dispatch_expand_s<YT, 2>(p, pl, grid, s); break;
    case 4: dispatch_expand_s<YT, 4>(p, pl, grid, s); break;
    case 8: dispatch_expand_s<YT, 8>(p, pl, grid, s); break;
    default: dispatch_expand_s<YT, 16>(p, pl, grid, s); break;
  }
}

// Kernel parameters of a decode-path call (both of its launches read them);
// `tiles` = the expand kernel's row tiles.
int build_mfma_params(const ProjDesc* pd, int np, const Plan& pl, int64_t M, int64_t K, const void* x,
                      const InputDesc& in, void* workspace, MfmaParams& p, int& tiles) {
  const int rows = 16 * (pl.waves / pl.splits);
  memset(&p, 0, sizeof(p));
  p.nproj = np;
  p.splits = pl.splits;
  p.ks = pl.ks;
  p.M = int(M);
  p.K = int(K);
  p.KW = int(ceil_div(K, 32));
  p.xmode = in.kind;
  p.x1 = in.x1;
  p.nw = in.nw;
  p.eps = in.eps;
  p.apos = in.pos_device;
  p.apos_host = in.pos;
  p.ahd = in.head_dim;
  p.amax_seq = in.max_seq;
  p.achunks = in.kind == LBK_INPUT_ATTN_MERGE ? int(ceil_div(in.max_seq, kAttnChunk)) : 0;
  bool xvec = (K % 8) == 0 && aligned16(x) && (!in.x1 || aligned16(in.x1)) && (!in.nw || aligned16(in.nw));
  bool wvec = true;
  int rb = 0, tbase = 0, si = 0, tile = 0;
  for (int q = 0; q < np; ++q) {
    ExpProj& P = p.proj[q];
    P.nb = pd[q].nb;
    P.N = int(pd[q].N);
    P.bias = pd[q].bias;
    P.res = pd[q].res;
    P.y = pd[q].y;
    P.tile0 = tile;
    tile += int(ceil_div(pd[q].N, rows));
    for (int b = 0; b < pd[q].nb; ++b, ++si) {
      const lbk_branch& B = pd[q].br[b];
      LatSeg& S = p.seg[si];
      S.V = reinterpret_cast<const uint32_t*>(B.v_sign);
      S.Vt = reinterpret_cast<const uint32_t*>(B.v_sign_tiled);
      S.g = B.v2;
      S.l = B.mid;
      S.R = int(B.rank);
      const int RW = int(ceil_div(B.rank, 32));
      const int RWp = int(ceil_div(RW, 4) * 4);
      S.RP = 32 * RWp;
      S.rb0 = rb;
      S.tbase = tbase;
      P.U[b] = reinterpret_cast<const uint32_t*>(B.u_sign);
      P.h[b] = B.u1;
      P.RW[b] = RW;
      P.RWp[b] = RWp;
      P.RP[b] = S.RP;
      P.tbase[b] = tbase;
      rb += int(ceil_div(B.rank, kRowBlock));
      tbase += int(M) * S.RP;
      wvec = wvec && (B.v_sign_tiled || (reinterpret_cast<uintptr_t>(B.v_sign) % 16) == 0);
      xvec = xvec && (reinterpret_cast<uintptr_t>(B.v2) % 16) == 0;
    }
  }
  p.nseg = si;
  p.tsize = tbase;
  p.nkc = pl.nkc;
  p.kc_major = 1;
  for (int i = 0; i < si; ++i) p.kc_major = p.kc_major && p.seg[i].Vt ? 1 : 0;
  // rows past the plan's tile (a call planned in row chunks): the chunks run
  // side by side in the same two launches
  p.crows = pl.chunk > 0 ? pl.chunk : int(M);
  p.x = x;
  p.wvec = wvec && p.KW % std::max(pl.wpl, 4) == 0 ? 1 : 0;
  p.xvec = xvec ? 1 : 0;
  p.late_rs = xvec && in.kind == LBK_INPUT_RMSNORM ? 1 : 0;
  if (in.kind == LBK_INPUT_ATTN_MERGE && (!xvec || M != 1))
    return set_error(LBK_ERR_ARG, "LBK_INPUT_ATTN_MERGE needs one row and 16-byte aligned g of every branch");
  char* ws = static_cast<char*>(workspace);
  p.sync = reinterpret_cast<uint32_t*>(ws);
  p.t2 = reinterpret_cast<float*>(ws + kTOffset);
  // the plan sized the workspace for the partials when the mode was on
  const bool det = pl.det && pl.nkc > 1 && pl.ws_min > kTOffset + kTBytes;
  p.part = det ? reinterpret_cast<float*>(ws + kGemmOffset) : nullptr;
  p.det_cnt = det ? reinterpret_cast<uint32_t*>(ws + kDetCntOffset) : nullptr;
  p.ntiles = tile;
  tiles = tile;
  return LBK_OK;
}

int forward_mfma(const ProjDesc* pd, int np, const Plan& pl, int64_t M, int64_t K, const void* x, int x_dtype,
                 const InputDesc& in, int y_dtype, void* workspace, hipStream_t s) {
  MfmaParams p;
  int tile = 0;
  int rc = build_mfma_params(pd, np, pl, M, K, x, in, workspace, p, tile);
  if (rc != LBK_OK) return rc;
  const int nchunks = int(ceil_div(M, p.crows));
  const dim3 grid1(unsigned(pl.nrb * pl.nkc), unsigned(nchunks));
  if (x_dtype == LBK_F32) dispatch_latent<float>(p, pl, grid1, s);
  else dispatch_latent<uint16_t>(p, pl, grid1, s);
  rc = check_launch("latent_mfma_kernel");
  if (rc != LBK_OK) return rc;

  // With slices, grid.x is padded to a multiple of the 8 XCDs (blocks are
  // dealt to the XCDs in turn by linear index), so that every slice of a
  // row tile runs on one XCD: U rows cut between slices share 128-byte lines,
  // which one L2 then fetches once instead of once per slice's XCD.
  const dim3 grid2(unsigned(pl.ks > 1 ? (tile + 7) / 8 * 8 : tile), unsigned(pl.ks), unsigned(nchunks));
  if (y_dtype == LBK_F32) dispatch_expand<float>(p, pl, grid2, s);
  else dispatch_expand<uint16_t>(p, pl, grid2, s);
  return check_launch("expand_mfma_kernel");
}

int forward_gemm(const ProjDesc* pd, int np, int64_t M, int64_t K, const void* x, int x_dtype, const InputDesc& in,
                 int y_dtype, void* workspace, size_t workspace_bytes, hipStream_t s) {
  const bool split = x_dtype == LBK_F32;
  GemmParams p;
  memset(&p, 0, sizeof(p));
  p.nproj = np;
  p.M = int(M);
  p.K = int(K);
  p.KW = int(ceil_div(K, 32));
  p.Kp = int(ceil_div(K, kGK) * kGK);
  p.x = x;
  gemm_planes(pd, np, M, K, p.a_plane, p.t_plane);
  char* ws = static_cast<char*>(workspace) + kGemmOffset;
  p.a = reinterpret_cast<uint16_t*>(ws);
  p.t = reinterpret_cast<uint16_t*>(ws + align256(size_t(p.a_plane) * (split ? 2 : 1) * sizeof(uint16_t)));
  p.xmode = in.kind;
  p.x1 = in.x1;
  p.nw = in.nw;
  p.eps = in.eps;
  bool xvec = (K % 8) == 0 && aligned16(x) && (!in.x1 || aligned16(in.x1)) && (!in.nw || aligned16(in.nw));
  int si = 0, nt1 = 0, nt2 = 0;
  int64_t abase = 0, tbase = 0;
  for (int q = 0; q < np; ++q) {
    GemmProj& P = p.proj[q];
    P.nb = pd[q].nb;
    P.N = int(pd[q].N);
    P.bias = pd[q].bias;
    P.res = pd[q].res;
    P.y = pd[q].y;
    P.nt0 = nt2;
    nt2 += int(ceil_div(pd[q].N, kGB));
    for (int b = 0; b < pd[q].nb; ++b, ++si) {
      const lbk_branch& B = pd[q].br[b];
      GemmSeg& S = p.seg[si];
      S.V = reinterpret_cast<const uint32_t*>(B.v_sign);
      S.g = B.v2;
      S.l = B.mid;
      S.R = int(B.rank);
      S.RP = int(ceil_div(B.rank, kGB) * kGB);
      S.nt0 = nt1;
      S.abase = abase;
      S.tbase = tbase;
      nt1 += S.RP / kGB;
      abase += M * p.Kp;
      P.U[b] = reinterpret_cast<const uint32_t*>(B.u_sign);
      P.h[b] = B.u1;
      P.RW[b] = int(ceil_div(B.rank, 32));
      P.RP[b] = S.RP;
      P.tbase[b] = tbase;
      tbase += M * S.RP;
      xvec = xvec && (reinterpret_cast<uintptr_t>(B.v2) % 16) == 0;
    }
  }
  p.nseg = si;
  p.xvec = xvec ? 1 : 0;
  const int64_t mtiles = ceil_div(M, kGB);
  if (nt1 > 65535 || nt2 > 65535) return set_error(LBK_ERR_ARG, "too many column tiles for the GEMM path");
  const size_t lds = 0;  // the stage ring is static LDS
  const dim3 g0{unsigned(M), unsigned(si), 1u};
  const dim3 g1{unsigned(mtiles), unsigned(nt1), 1u}, g2{unsigned(mtiles), unsigned(nt2), 1u};
  // bf16 rows of whole k-steps, taken as they are: g goes into stage 1's B
  // operand and no scaled copy of x is made
  const bool direct = !split && in.kind == LBK_INPUT_PLAIN && K % kGK == 0 && aligned16(x);
  // Stream-K stage 1 when whole tiles would leave the block slots unevenly
  // used (estimated in k-steps of one block: rounds of tiles vs an even
  // share plus about two steps for the partial tiles), and the workspace
  // holds the partial tiles.
  const int64_t nks = p.Kp / kGK, tiles = mtiles * nt1;
  const int slots = (split ? 1 : 2) * kNumCUs;  // blocks resident at once (LDS of the stage ring)
  const size_t part_off = kGemmOffset + gemm_ws_bytes(pd, np, M, K, true);
  const int64_t P = sk_blocks(tiles, nks, slots);
  const bool sk = P > 0 && workspace_bytes >= part_off + size_t(2 * P) * kSkSlotBytes;
  SkParams q{};
  q.G = mtiles % 8 == 0 && P % 8 == 0 ? 8 : 1;
  q.P = int(std::max<int64_t>(P, 1)) / q.G;
  q.NT = nt1;
  q.nks = int(nks);
  q.W = tiles / q.G * nks;
  q.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + part_off);
  q.cnt = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + kSkCntOffset);
  const dim3 gsk{unsigned(q.G * q.P), 1u, 1u};
  int rc;
  if (direct) {
    p.a = const_cast<uint16_t*>(static_cast<const uint16_t*>(x));
    for (int i = 0; i < si; ++i) p.seg[i].abase = 0;
    if (sk) hipLaunchKernelGGL((gemm_latent_sk_kernel<false, true>), gsk, dim3(kGThreads), 0, s, p, q);
    else hipLaunchKernelGGL((gemm_latent_kernel<false, true>), g1, dim3(kGThreads), lds, s, p);
  } else {
    if (x_dtype == LBK_F32) hipLaunchKernelGGL((gemm_scale_kernel<float, true>), g0, dim3(kGThreads), 0, s, p);
    else hipLaunchKernelGGL((gemm_scale_kernel<uint16_t, false>), g0, dim3(kGThreads), 0, s, p);
    rc = check_launch("gemm_scale_kernel");
    if (rc != LBK_OK) return rc;
    if (split) {
      if (sk) hipLaunchKernelGGL((gemm_latent_sk_kernel<true, false>), gsk, dim3(kGThreads), 0, s, p, q);
      else hipLaunchKernelGGL((gemm_latent_kernel<true, false>), g1, dim3(kGThreads), lds, s, p);
    } else {
      if (sk) hipLaunchKernelGGL((gemm_latent_sk_kernel<false, false>), gsk, dim3(kGThreads), 0, s, p, q);
      else hipLaunchKernelGGL((gemm_latent_kernel<false, false>), g1, dim3(kGThreads), lds, s, p);
    }
  }
  rc = check_launch("gemm_latent_kernel");
  if (rc != LBK_OK) return rc;
  if (split) {
    if (y_dtype == LBK_F32) hipLaunchKernelGGL((gemm_expand_kernel<float, true>), g2, dim3(kGThreads), lds, s, p);
    else hipLaunchKernelGGL((gemm_expand_kernel<uint16_t, true>), g2, dim3(kGThreads), lds, s, p);
    return check_launch("gemm_expand_kernel");
  }
  // bf16 activations: 256-column tiles where they still give every CU two
  // blocks (the stage ring allows two per CU); else 128-column tiles
  int ntw = 0;
  for (int q = 0; q < np; ++q) ntw += int(ceil_div(pd[q].N, 2 * kGB));
  if (mtiles * ntw >= 2 * kNumCUs && ntw <= 65535) {
    for (int q = 0, t = 0; q < np; ++q) {
      p.proj[q].nt0 = t;
      t += int(ceil_div(pd[q].N, 2 * kGB));
    }
    const dim3 gw{unsigned(mtiles), unsigned(ntw), 1u};
    if (y_dtype == LBK_F32) hipLaunchKernelGGL((gemm_expand_wide_kernel<float>), gw, dim3(kGThreads), lds, s, p);
    else hipLaunchKernelGGL((gemm_expand_wide_kernel<uint16_t>), gw, dim3(kGThreads), lds, s, p);
    return check_launch("gemm_expand_wide_kernel");
  }
  if (y_dtype == LBK_F32) hipLaunchKernelGGL((gemm_expand_kernel<float, false>), g2, dim3(kGThreads), lds, s, p);
  else hipLaunchKernelGGL((gemm_expand_kernel<uint16_t, false>), g2, dim3(kGThreads), lds, s, p);
  return check_launch("gemm_expand_kernel");
}

bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
  return a && b && na && nb && a0 < b0 + nb && b0 < a0 + na;
}

// Whether the expand stage may cut the rank into slices (plan_one's
// allow_ks): the slices add to y with fp32 atomics after the latent kernel
// has set y = bias + residual, so y must be fp32, the mode not deterministic,
// and no y may overlap what the latent kernel reads (x, x1).
bool slices_allowed(const ProjDesc* pd, int np, int64_t M, int64_t K, const void* x, int x_dtype,
                    const InputDesc& in, int y_dtype, bool det) {
  if (y_dtype != LBK_F32 || det) return false;
  const size_t xb = x_dtype == LBK_F32 ? 4 : 2;
  size_t xbytes = size_t(M) * size_t(K) * xb;
  if (in.kind == LBK_INPUT_ATTN_MERGE)  // partials [K / head_dim][chunks][head_dim + 4] fp32
    xbytes = size_t(K / in.head_dim) * size_t(ceil_div(in.max_seq, kAttnChunk)) * size_t(in.head_dim + 4) * 4;
  for (int q = 0; q < np; ++q) {
    const size_t ybytes = size_t(M) * size_t(pd[q].N) * 4;
    if (overlaps(pd[q].y, ybytes, x, xbytes) || overlaps(pd[q].y, ybytes, in.x1, size_t(M) * size_t(K) * xb))
      return false;
  }
  return true;
}

// Workspace a call of these shapes needs whatever its output dtype and
// buffers (with or without rank slices).
size_t query_workspace(const ProjDesc* pd, int np, int64_t M, int64_t K) {
  const bool det = g_deterministic.load() != 0;
  const Plan a = make_plan(pd, np, M, K, false, det);
  if (det) return a.ws_total;
  return std::max(a.ws_total, make_plan(pd, np, M, K, true, det).ws_total);
}

// Chunks run one after another (Plan::seq): chunk c reads rows [c * ch,
// (c + 1) * ch) of x, x1 and each residual, then writes the same rows of
// each y.  An output overlapping an input row that a later chunk still has
// to read would change that chunk's input, so the chunks run in an order
// in which no chunk's output rows overlap the input rows of any chunk after
// it: first to last, else last to first (e.g. y at x's address with wider
// rows than x), else the call is refused.
bool chunk_order_safe(const ProjDesc* pd, int np, int64_t M, int64_t K, int64_t ch, const void* x, size_t xb,
                      const void* x1, int y_dtype, bool reverse) {
  const size_t yb = y_dtype == LBK_F32 ? 4 : 2;
  const int64_t nc = ceil_div(M, ch);
  auto rows = [&](int64_t c, int64_t& m0, int64_t& mc) {
    m0 = c * ch;
    mc = std::min<int64_t>(ch, M - m0);
  };
  for (int64_t i = 0; i < nc; ++i) {
    int64_t m0, mc;
    rows(i, m0, mc);
    for (int q = 0; q < np; ++q) {
      const char* y = static_cast<const char*>(pd[q].y) + size_t(m0) * size_t(pd[q].N) * yb;
      const size_t ybytes = size_t(mc) * size_t(pd[q].N) * yb;
      for (int64_t j = reverse ? 0 : i + 1; j < (reverse ? i : nc); ++j) {
        int64_t n0, nn;
        rows(j, n0, nn);
        const size_t xo = size_t(n0) * size_t(K) * xb, xn = size_t(nn) * size_t(K) * xb;
        if (overlaps(y, ybytes, static_cast<const char*>(x) + xo, xn)) return false;
        if (x1 && overlaps(y, ybytes, static_cast<const char*>(x1) + xo, xn)) return false;
        for (int r = 0; r < np; ++r) {
          if (!pd[r].res) continue;
          const float* res = pd[r].res + size_t(n0) * size_t(pd[r].N);
          if (overlaps(y, ybytes, res, size_t(nn) * size_t(pd[r].N) * 4)) return false;
        }
      }
    }
  }
  return true;
}

// Validation and plan of a group call, without touching the device; M == 0
// leaves pl.mfma false and pl.ws_min 0 (nothing to run).
int prepare_group(const ProjDesc* pd, int np, int64_t M, int64_t K, const void* x, int x_dtype,
                  const lbk_input* input, int y_dtype, InputDesc& in, Plan& pl) {
  int rc = validate_group(pd, np, M, K);
  if (rc != LBK_OK) return rc;
  pl = Plan{};
  in = InputDesc{LBK_INPUT_PLAIN, nullptr, 0.f, nullptr, 0, 0, nullptr, 0};
  if (input) {
    in = InputDesc{input->kind, input->rms_weight, input->rms_eps, input->x1,
                   0, 0, nullptr, 0};
    if (in.kind == LBK_INPUT_ATTN_MERGE) {
      in.nw = nullptr;
      in.x1 = nullptr;
      in.head_dim = input->head_dim;
      in.max_seq = input->max_seq;
      in.pos_device = input->pos_device;
      in.pos = input->pos;
      if (M != 1 && M != 0) return set_error(LBK_ERR_ARG, "LBK_INPUT_ATTN_MERGE needs M == 1, got %lld", (long long)M);
      if (x_dtype != LBK_F32) return set_error(LBK_ERR_DTYPE, "LBK_INPUT_ATTN_MERGE reads fp32 partials");
      if (in.head_dim != 64 && in.head_dim != 128)
        return set_error(LBK_ERR_ARG, "LBK_INPUT_ATTN_MERGE: head_dim must be 64 or 128, got %d", in.head_dim);
      if (K % in.head_dim != 0)
        return set_error(LBK_ERR_ARG, "LBK_INPUT_ATTN_MERGE: K (%lld) must be heads * head_dim", (long long)K);
      if (in.max_seq < 1 || in.max_seq > (1 << 24))
        return set_error(LBK_ERR_ARG, "LBK_INPUT_ATTN_MERGE: max_seq out of range: %d", in.max_seq);
      if (x && !aligned16(x)) return set_error(LBK_ERR_ARG, "LBK_INPUT_ATTN_MERGE: partials must be 16-byte aligned");
    } else if (in.kind == LBK_INPUT_RMSNORM) {
      if (!in.nw) return set_error(LBK_ERR_ARG, "LBK_INPUT_RMSNORM needs rms_weight");
      if (!(in.eps >= 0.f)) return set_error(LBK_ERR_ARG, "rms_eps must be >= 0");
      in.x1 = nullptr;
    } else if (in.kind == LBK_INPUT_SILU_MUL) {
      if (!in.x1) return set_error(LBK_ERR_ARG, "LBK_INPUT_SILU_MUL needs x1");
      in.nw = nullptr;
    } else if (in.kind == LBK_INPUT_PLAIN) {
      in.nw = nullptr;
      in.x1 = nullptr;
    } else {
      return set_error(LBK_ERR_ARG, "input kind %d unknown", in.kind);
    }
  }
  if (x_dtype != LBK_F32 && x_dtype != LBK_BF16) return set_error(LBK_ERR_DTYPE, "x_dtype %d unsupported", x_dtype);
  if (y_dtype != LBK_F32 && y_dtype != LBK_BF16) return set_error(LBK_ERR_DTYPE, "y_dtype %d unsupported", y_dtype);
  if (M == 0) return LBK_OK;
  if (!x) return set_error(LBK_ERR_ARG, "x is NULL");
  for (int q = 0; q < np; ++q)
    if (!pd[q].y) return set_error(LBK_ERR_ARG, "projection %d: y is NULL", q);
  const bool det = g_deterministic.load() != 0;
  pl = make_plan(pd, np, M, K, slices_allowed(pd, np, M, K, x, x_dtype, in, y_dtype, det), det);
  if (pl.chunk > 0 && pl.seq) {
    const size_t xb = x_dtype == LBK_F32 ? 4 : 2;
    if (!chunk_order_safe(pd, np, M, K, pl.chunk, x, xb, in.x1, y_dtype, false)) {
      if (!chunk_order_safe(pd, np, M, K, pl.chunk, x, xb, in.x1, y_dtype, true))
        return set_error(LBK_ERR_ARG,
                         "an output overlaps input rows of other row chunks (%lld rows run as chunks of %d): "
                         "pass an output that does not share memory with the input",
                         (long long)M, pl.chunk);
      pl.reverse = true;
    }
  }
  if (in.kind == LBK_INPUT_ATTN_MERGE && (!pl.mfma || pl.chunk > 0))
    return set_error(LBK_ERR_ARG, "LBK_INPUT_ATTN_MERGE: the projections have no one-row decode plan");
  return LBK_OK;
}

// Launch a prepared call on the workspace.
int run_group(const ProjDesc* pd, int np, int64_t M, int64_t K, const void* x, int x_dtype, const InputDesc& in,
              int y_dtype, const Plan& pl, void* workspace, size_t workspace_bytes, void* stream) {
  if (M == 0) return LBK_OK;
  int rc = LBK_OK;
  if (!workspace || workspace_bytes < pl.ws_min)
    return set_error(LBK_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", pl.ws_min, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (pl.chunk > 0 && !pl.seq) {
    // every chunk's t fits the latent half: the chunks run side by side in
    // one launch pair (each block takes one chunk's rows)
    return forward_mfma(pd, np, pl, M, K, x, x_dtype, in, y_dtype, workspace, s);
  }
  if (pl.chunk > 0) {
    // one launch pair per chunk (deterministic mode sizes its partials for
    // one chunk; or the rows' t does not fit the latent half at once)
    const size_t xb = x_dtype == LBK_F32 ? 4 : 2, yb = y_dtype == LBK_F32 ? 4 : 2;
    const int64_t nc = ceil_div(M, pl.chunk);
    for (int64_t i = 0; i < nc; ++i) {
      const int64_t m0 = (pl.reverse ? nc - 1 - i : i) * pl.chunk;
      const int64_t mc = std::min<int64_t>(pl.chunk, M - m0);
      ProjDesc pc[kMaxProj];
      for (int q = 0; q < np; ++q) {
        pc[q] = pd[q];
        pc[q].y = static_cast<char*>(pd[q].y) + size_t(m0) * size_t(pd[q].N) * yb;
        if (pd[q].res) pc[q].res = pd[q].res + size_t(m0) * size_t(pd[q].N);
      }
      InputDesc ic = in;
      if (ic.x1) ic.x1 = static_cast<const char*>(in.x1) + size_t(m0) * size_t(K) * xb;
      const Plan pm = plan_one(pc, np, mc, K, pl.allow_ks, pl.det);
      if (!pm.mfma) return set_error(LBK_ERR_ARG, "a chunk of %lld rows has no decode-path plan", (long long)mc);
      if (pm.ws_min > workspace_bytes)
        return set_error(LBK_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", pm.ws_min, workspace_bytes);
      rc = forward_mfma(pc, np, pm, mc, K, static_cast<const char*>(x) + size_t(m0) * size_t(K) * xb, x_dtype, ic,
                        y_dtype, workspace, s);
      if (rc != LBK_OK) return rc;
    }
    return LBK_OK;
  }
  if (pl.mfma) return forward_mfma(pd, np, pl, M, K, x, x_dtype, in, y_dtype, workspace, s);
  return forward_gemm(pd, np, M, K, x, x_dtype, in, y_dtype, workspace, workspace_bytes, s);
}

int forward_group(const ProjDesc* pd, int np, int64_t M, int64_t K, const void* x, int x_dtype,
                  const lbk_input* input, int y_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  InputDesc in;
  Plan pl;
  const int rc = prepare_group(pd, np, M, K, x, x_dtype, input, y_dtype, in, pl);
  if (rc != LBK_OK) return rc;
  return run_group(pd, np, M, K, x, x_dtype, in, y_dtype, pl, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Chains on the host (see chain_mfma_kernel)
// ---------------------------------------------------------------------------
struct ChainLinkDesc {
  ProjDesc pd[kMaxProj];
  int np;
  int64_t K;
  const void* x;  // link 0: the caller's input; then projection 0's y of the link before
  InputDesc in;
  Plan pl;
};

template <int S, int W, int NT>
void launch_chain(const ChainParams& cp, unsigned blocks, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((chain_mfma_kernel<S, W, NT>), dim3(blocks), dim3(W * kWave), lds, s, cp);
}
template <int S, int W>
void dispatch_chain_nt(const ChainParams& cp, int nt, unsigned blocks, size_t lds, hipStream_t s) {
  if (nt == 2) launch_chain<S, W, 2>(cp, blocks, lds, s);
  else launch_chain<S, W, 1>(cp, blocks, lds, s);
}
template <int S>
void dispatch_chain_w(const ChainParams& cp, int w, int nt, unsigned blocks, size_t lds, hipStream_t s) {
  (void)w;  // chain_waves: 8
  dispatch_chain_nt<S, 8>(cp, nt, blocks, lds, s);
}
void dispatch_chain(const ChainParams& cp, int steps, int w, int nt, unsigned blocks, size_t lds, hipStream_t s) {
  switch (steps) {
    case 4: dispatch_chain_w<4>(cp, w, nt, blocks, lds, s); break;
    case 8: dispatch_chain_w<8>(cp, w, nt, blocks, lds, s); break;
    default: dispatch_chain_w<16>(cp, w, nt, blocks, lds, s); break;
  }
}

constexpr int kChainMaxSteps = 16;  // rank steps of a joined link's projection (both branches)

// Waves of the kernel joining a link with N outputs to the next: 16 W rows
// per block, so N / (16 W) blocks each add one partial latent vector.  At
// one row its waves are bound by their own instruction streams, so two per
// SIMD on more CUs beat four per SIMD on fewer (draft step 1.085 -> 1.049 ms
// against 16 waves above 8192 outputs; 4 waves: 1.171 ms).
int chain_waves(int64_t) { return 8; }

// Latent floats of a link at one row (every branch's RP), as build_mfma_params lays them out.
int64_t chain_tsize(const ProjDesc* pd, int np) {
  int64_t t = 0;
  for (int q = 0; q < np; ++q)
    for (int b = 0; b < pd[q].nb; ++b) t += 32 * ceil_div(ceil_div(pd[q].br[b].rank, 32), 4) * 4;
  return t;
}

// Validation and plans of a chain; `fused` tells whether it runs as one
// kernel per link boundary (else every link runs as its own call).
int prepare_chain(const lbk_chain_link* links, int n, const void* x, ChainLinkDesc* cl, bool& fused) {
  if (!links || n < 1 || n > kMaxChainLinks)
    return set_error(LBK_ERR_ARG, "n_links must be in [1, %d] with a non-NULL array, got %d", kMaxChainLinks, n);
  for (int j = 0; j < n; ++j) {
    const lbk_chain_link& lk = links[j];
    ChainLinkDesc& c = cl[j];
    if (!lk.projs || lk.n_proj < 1 || lk.n_proj > kMaxProj)
      return set_error(LBK_ERR_ARG, "link %d: n_proj must be in [1, %d] with a non-NULL array, got %d", j, kMaxProj,
                       lk.n_proj);
    c.np = lk.n_proj;
    c.K = lk.in_features;
    for (int q = 0; q < c.np; ++q)
      c.pd[q] = ProjDesc{lk.projs[q].branches, lk.projs[q].n_branches, lk.projs[q].out_features, lk.projs[q].bias,
                         lk.projs[q].y, lk.projs[q].residual};
    lbk_input inp{};
    inp.kind = LBK_INPUT_PLAIN;
    if (lk.input) inp = *lk.input;
    c.x = x;
    if (j > 0) {
      const ChainLinkDesc& pv = cl[j - 1];
      if (inp.kind == LBK_INPUT_SILU_MUL) {
        if (pv.np != 2)
          return set_error(LBK_ERR_ARG, "link %d reads SiLU(gate) * up: link %d must have two projections, has %d", j,
                           j - 1, pv.np);
        inp.x1 = pv.pd[1].y;
      } else if (inp.kind == LBK_INPUT_PLAIN || inp.kind == LBK_INPUT_RMSNORM) {
        if (pv.np != 1)
          return set_error(LBK_ERR_ARG, "link %d reads the output of link %d, which must have one projection, has %d",
                           j, j - 1, pv.np);
      } else {
        return set_error(LBK_ERR_ARG, "link %d: input kind %d cannot follow a link (plain, RMSNorm or SiLU * up)", j,
                         inp.kind);
      }
      for (int q = 0; q < pv.np; ++q)
        if (pv.pd[q].N != c.K)
          return set_error(LBK_ERR_ARG, "link %d: in_features %lld != out_features %lld of link %d", j,
                           (long long)c.K, (long long)pv.pd[q].N, j - 1);
      c.x = pv.pd[0].y;
    }
    const int rc = prepare_group(c.pd, c.np, 1, c.K, c.x, LBK_F32, &inp, LBK_F32, c.in, c.pl);
    if (rc != LBK_OK) {
      char msg[sizeof(g_last_error)];
      snprintf(msg, sizeof(msg), "%s", g_last_error);
      return set_error(rc, "link %d: %s", j, msg);
    }
  }
  fused = n >= 2 && !cl[0].pl.det;
  for (int j = 0; j < n && fused; ++j) {
    const ChainLinkDesc& c = cl[j];
    fused = c.pl.mfma && c.pl.mt == 1 && c.pl.chunk == 0 && c.pl.ks == 1 &&
            chain_tsize(c.pd, c.np) + kSsqSlots <= kChainRegion;
    if (!fused || j == 0) continue;
    // joined to the link before: 16-byte loads of g (and the RMSNorm
    // weight) by 8-column chunks, V read from its tiled copy, the link
    // before's steps within the kernel's bound, its staged t and this
    // link's A operand within LDS
    fused = c.K % 8 == 0 && (c.in.kind != LBK_INPUT_RMSNORM || aligned16(c.in.nw));
    for (int q = 0; q < c.np && fused; ++q)
      for (int b = 0; b < c.pd[q].nb; ++b)
        fused = fused && aligned16(c.pd[q].br[b].v2) && c.pd[q].br[b].v_sign_tiled;
    const ChainLinkDesc& pv = cl[j - 1];
    int64_t chunks = 0;
    for (int q = 0; q < pv.np && fused; ++q) {
      fused = proj_steps(pv.pd[q]) <= kChainMaxSteps;
      for (int b = 0; b < pv.pd[q].nb; ++b) chunks += 16 * ceil_div(ceil_div(pv.pd[q].br[b].rank, 32), 4);
    }
    int nseg = 0;
    for (int q = 0; q < c.np; ++q) nseg += c.pd[q].nb;
    const int w = chain_waves(pv.pd[0].N);
    fused = fused && nseg <= w && size_t(chunks + int64_t(nseg) * 2 * w) * 48 <= 64 * 1024;
  }
  return LBK_OK;
}

size_t chain_ws_bytes(const ChainLinkDesc* cl, int n, bool fused) {
  size_t ws = fused ? kGemmOffset : 0;
  for (int j = 0; j < n; ++j) ws = std::max(ws, cl[j].pl.ws_min);
  return ws;
}

int run_chain(ChainLinkDesc* cl, int n, bool fused, void* workspace, size_t workspace_bytes, void* stream) {
  const size_t need = chain_ws_bytes(cl, n, fused);
  if (!workspace || workspace_bytes < need)
    return set_error(LBK_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!fused) {
    for (int j = 0; j < n; ++j) {
      const ChainLinkDesc& c = cl[j];
      const int rc = run_group(c.pd, c.np, 1, c.K, c.x, LBK_F32, c.in, LBK_F32, c.pl, workspace, workspace_bytes,
                               stream);
      if (rc != LBK_OK) return rc;
    }
    return LBK_OK;
  }
  float* regions = reinterpret_cast<float*>(static_cast<char*>(workspace) + kChainOffset);
  auto region = [&](int i) { return regions + size_t(i) * kChainRegion; };
  auto target = [&](int j) { return j == n - 1 ? region(kChainLast) : region(j); };  // region holding link j's t
  // link 0's latent stage
  {
    const ChainLinkDesc& c = cl[0];
    MfmaParams p;
    int tiles = 0;
    int rc = build_mfma_params(c.pd, c.np, c.pl, 1, c.K, c.x, c.in, workspace, p, tiles);
    if (rc != LBK_OK) return rc;
    p.tdst = target(0);
    p.clr = region(kChainLast);
    p.nclr = kChainRegion;
    dispatch_latent<float>(p, c.pl, dim3(unsigned(c.pl.nrb * c.pl.nkc), 1u), s);
    rc = check_launch("latent_mfma_kernel");
    if (rc != LBK_OK) return rc;
  }
  // link j's expand joined to link j + 1's latent stage
  for (int j = 0; j + 1 < n; ++j) {
    const ChainLinkDesc& a = cl[j];
    const ChainLinkDesc& b = cl[j + 1];
    MfmaParams pe, pb;
    int tiles = 0;
    int rc = build_mfma_params(a.pd, a.np, a.pl, 1, a.K, a.x, a.in, workspace, pe, tiles);
    if (rc != LBK_OK) return rc;
    rc = build_mfma_params(b.pd, b.np, b.pl, 1, b.K, b.x, b.in, workspace, pb, tiles);
    if (rc != LBK_OK) return rc;
    ChainParams cp;
    memset(&cp, 0, sizeof(cp));
    cp.tsrc = target(j);
    cp.tdst = target(j + 1);
    cp.nw = pb.nw;
    cp.clr = j > 0 ? region(j - 1) : nullptr;
    cp.nclr = j > 0 ? int(chain_tsize(cl[j - 1].pd, cl[j - 1].np)) + kSsqSlots : 0;
    cp.tsize_e = pe.tsize;
    // link 0's latent kernel applied 1/rms itself unless it deferred it; a
    // joined kernel always defers it
    cp.late = j > 0 ? (a.in.kind == LBK_INPUT_RMSNORM ? 1 : 0) : pe.late_rs;
    cp.Ke = pe.K;
    cp.N = pe.proj[0].N;
    cp.eps = pe.eps;
    cp.nseg = pb.nseg;
    cp.Kl = pb.K;
    cp.KWl = pb.KW;
    cp.xmode = b.in.kind;
    cp.tsize_l = pb.tsize;
    for (int q = 0; q < a.np && q < 2; ++q) {
      const ExpProj& P = pe.proj[q];
      ChainProj& C = cp.proj[q];
      for (int br = 0; br < 2; ++br) {
        C.U[br] = P.U[br];
        C.h[br] = P.h[br];
        C.RW[br] = P.RW[br];
        C.steps[br] = P.RWp[br] / 4;
        C.tbase[br] = P.tbase[br];
      }
      C.bias = P.bias;
      C.res = P.res;
      C.y = static_cast<float*>(P.y);
      C.nb = P.nb;
    }
    for (int i = 0; i < pb.nseg; ++i)
      cp.seg[i] = ChainSeg{pb.seg[i].Vt, pb.seg[i].l, pb.seg[i].g, pb.seg[i].R, pb.seg[i].tbase};
    const int nt = b.in.kind == LBK_INPUT_SILU_MUL ? 2 : 1;
    int64_t steps = 0, chunks = 0;
    for (int q = 0; q < nt; ++q) {
      steps = std::max(steps, proj_steps(a.pd[q]));
      for (int br = 0; br < a.pd[q].nb; ++br) chunks += 16 * ceil_div(ceil_div(a.pd[q].br[br].rank, 32), 4);
    }
    const int w = chain_waves(a.pd[0].N);
    const size_t lds = size_t(chunks + int64_t(cp.nseg) * 2 * w) * 48;
    const unsigned blocks = unsigned(ceil_div(a.pd[0].N, int64_t(16 * w)));
    dispatch_chain(cp, steps <= 4 ? 4 : steps <= 8 ? 8 : 16, w, nt, blocks, lds, s);
    rc = check_launch("chain_mfma_kernel");
    if (rc != LBK_OK) return rc;
  }
  // link n - 1's expand stage
  {
    const ChainLinkDesc& c = cl[n - 1];
    MfmaParams p;
    int tiles = 0;
    int rc = build_mfma_params(c.pd, c.np, c.pl, 1, c.K, c.x, c.in, workspace, p, tiles);
    if (rc != LBK_OK) return rc;
    p.late_rs = c.in.kind == LBK_INPUT_RMSNORM ? 1 : 0;  // the joined kernel left 1/rms out
    p.tsrc = target(n - 1);
    p.clr = region(n - 2);
    p.nclr = int(chain_tsize(cl[n - 2].pd, cl[n - 2].np)) + kSsqSlots;
    dispatch_expand<float>(p, c.pl, dim3(unsigned(tiles), 1u, 1u), s);
    return check_launch("expand_mfma_kernel");
  }
}

// ---------------------------------------------------------------------------
// Allocation-free forward: the workspace is a file-scope device array.
// Each GPU the library runs on holds its own copy of `scratch` until the
// process ends.  In host code `scratch` names a host-side stand-in, not the
// device memory: the host takes each device's address once, with
// hipGetSymbolAddress, and passes only that address on.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = LBK_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes >= kTOffset + kTBytes, "scratch must hold the decode path's latent buffer and state");
static_assert(kScratchBytes % 16 == 0, "scratch is cleared in 16-byte stores");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ __launch_bounds__(kBlock) void clear_kernel(u32x4* __restrict__ p, int64_t n16) {
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n16; i += int64_t(gridDim.x) * kBlock)
    p[i] = u32x4{0u, 0u, 0u, 0u};
}

constexpr int kMaxDevices = 64;
struct ScratchSlot {
  void* ptr = nullptr;  // this device's `scratch`, from hipGetSymbolAddress
  bool clean = false;   // the latent-buffer state in it is consistent
};
std::mutex g_scratch_mu;
ScratchSlot g_scratch[kMaxDevices];

// The current device's scratch address; at its first use (and after a call
// that failed part-way) the scratch is zeroed by a kernel on `s`, ahead of
// the call's own kernels (a kernel, not hipMemsetAsync: the call may be
// captured into a graph).
int device_scratch(hipStream_t s, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(LBK_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(LBK_ERR_ARG, "device %d out of range [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchSlot& slot = g_scratch[dev];
  if (!slot.ptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(LBK_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                       hipGetErrorString(e));
    slot.ptr = ptr;
  }
  if (!slot.clean) {
    // A clear enqueued while `s` is being captured runs in every replay of
    // the graph and never now: the array stays marked unclean, so the next
    // eager call clears it again (a capture query that fails counts as a
    // capture).
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone;
    const int64_t n16 = int64_t(kScratchBytes / 16);
    hipLaunchKernelGGL(clear_kernel, dim3(unsigned(std::min<int64_t>(ceil_div(n16, kBlock), 2048))), dim3(kBlock), 0,
                       s, static_cast<u32x4*>(slot.ptr), n16);
    const int rc = check_launch("clear_kernel");
    if (rc != LBK_OK) return rc;
    if (!capturing) slot.clean = true;
  }
  *out = slot.ptr;
  return LBK_OK;
}

void scratch_dirty() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  g_scratch[dev].clean = false;
}

}  // namespace

extern "C" {

int lbk_abi_version(void) { return LBK_ABI_VERSION; }

const char* lbk_last_error(void) { return g_last_error; }

int lbk_set_deterministic(int on) { return g_deterministic.exchange(on ? 1 : 0); }

size_t lbk_group_workspace_bytes(const lbk_projection* projs, int n_proj, int64_t M, int64_t K) {
  ProjDesc pd[kMaxProj];
  if (!projs || n_proj < 1 || n_proj > kMaxProj) {
    set_error(LBK_ERR_ARG, "n_proj must be in [1, %d] with a non-NULL array, got %d", kMaxProj, n_proj);
    return 0;
  }
  for (int q = 0; q < n_proj; ++q)
    pd[q] = ProjDesc{projs[q].branches, projs[q].n_branches, projs[q].out_features, projs[q].bias, projs[q].y,
                     projs[q].residual};
  if (validate_group(pd, n_proj, M, K) != LBK_OK) return 0;
  return query_workspace(pd, n_proj, M, K);
}

int lbk_group_forward_ex(const lbk_projection* projs, int n_proj, int64_t M, int64_t K, const void* x, int x_dtype,
                         const lbk_input* input, int y_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error[0] = '\0';
  if (!projs || n_proj < 1 || n_proj > kMaxProj)
    return set_error(LBK_ERR_ARG, "n_proj must be in [1, %d] with a non-NULL array, got %d", kMaxProj, n_proj);
  ProjDesc pd[kMaxProj];
  for (int q = 0; q < n_proj; ++q)
    pd[q] = ProjDesc{projs[q].branches, projs[q].n_branches, projs[q].out_features, projs[q].bias, projs[q].y,
                     projs[q].residual};
  return forward_group(pd, n_proj, M, K, x, x_dtype, input, y_dtype, workspace, workspace_bytes, stream);
}

int lbk_group_forward_noalloc(const lbk_projection* projs, int n_proj, int64_t M, int64_t K, const void* x,
                              int x_dtype, const lbk_input* input, int y_dtype, void* stream) {
  g_last_error[0] = '\0';
  if (!projs || n_proj < 1 || n_proj > kMaxProj)
    return set_error(LBK_ERR_ARG, "n_proj must be in [1, %d] with a non-NULL array, got %d", kMaxProj, n_proj);
  ProjDesc pd[kMaxProj];
  for (int q = 0; q < n_proj; ++q)
    pd[q] = ProjDesc{projs[q].branches, projs[q].n_branches, projs[q].out_features, projs[q].bias, projs[q].y,
                     projs[q].residual};
  InputDesc in;
  Plan pl;
  int rc = prepare_group(pd, n_proj, M, K, x, x_dtype, input, y_dtype, in, pl);
  if (rc != LBK_OK) return rc;
  if (M == 0) return LBK_OK;
  if (pl.ws_min > kScratchBytes)
    return set_error(LBK_ERR_WORKSPACE,
                     "these shapes need %zu bytes of workspace; the allocation-free entry point's scratch holds "
                     "%zu (call lbk_group_forward_ex with a workspace instead)",
                     pl.ws_min, kScratchBytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  rc = device_scratch(s, &ws);
  if (rc != LBK_OK) return rc;
  rc = run_group(pd, n_proj, M, K, x, x_dtype, in, y_dtype, pl, ws, kScratchBytes, stream);
  if (rc == LBK_ERR_HIP) scratch_dirty();
  return rc;
}

size_t lbk_chain_workspace_bytes(const lbk_chain_link* links, int n_links) {
  g_last_error[0] = '\0';
  if (!links || n_links < 1 || n_links > kMaxChainLinks) {
    set_error(LBK_ERR_ARG, "n_links must be in [1, %d] with a non-NULL array, got %d", kMaxChainLinks, n_links);
    return 0;
  }
  // the decode-path workspace of each link, and the chains' regions
  size_t ws = kGemmOffset;
  for (int j = 0; j < n_links; ++j) {
    const lbk_chain_link& lk = links[j];
    if (!lk.projs || lk.n_proj < 1 || lk.n_proj > kMaxProj) {
      set_error(LBK_ERR_ARG, "link %d: n_proj must be in [1, %d] with a non-NULL array, got %d", j, kMaxProj,
                lk.n_proj);
      return 0;
    }
    ProjDesc pd[kMaxProj];
    for (int q = 0; q < lk.n_proj; ++q)
      pd[q] = ProjDesc{lk.projs[q].branches, lk.projs[q].n_branches, lk.projs[q].out_features, lk.projs[q].bias,
                       lk.projs[q].y, lk.projs[q].residual};
    if (validate_group(pd, lk.n_proj, 1, lk.in_features) != LBK_OK) return 0;
    ws = std::max(ws, query_workspace(pd, lk.n_proj, 1, lk.in_features));
  }
  return ws;
}

int lbk_chain_forward(const lbk_chain_link* links, int n_links, const void* x, void* workspace,
                      size_t workspace_bytes, void* stream) {
  g_last_error[0] = '\0';
  ChainLinkDesc cl[kMaxChainLinks];
  bool fused = false;
  const int rc = prepare_chain(links, n_links, x, cl, fused);
  if (rc != LBK_OK) return rc;
  return run_chain(cl, n_links, fused, workspace, workspace_bytes, stream);
}

int lbk_chain_fused(const lbk_chain_link* links, int n_links, const void* x) {
  g_last_error[0] = '\0';
  ChainLinkDesc cl[kMaxChainLinks];
  bool fused = false;
  const int rc = prepare_chain(links, n_links, x, cl, fused);
  if (rc != LBK_OK) return rc;
  return fused ? 1 : 0;
}

int lbk_group_forward(const lbk_projection* projs, int n_proj, int64_t M, int64_t K, const void* x, int x_dtype,
                      int y_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return lbk_group_forward_ex(projs, n_proj, M, K, x, x_dtype, nullptr, y_dtype, workspace, workspace_bytes, stream);
}

size_t lbk_linear_workspace_bytes(const lbk_branch* branches, int n_branches, int64_t M, int64_t K, int64_t N) {
  const ProjDesc pd{branches, n_branches, N, nullptr, nullptr, nullptr};
  if (validate_group(&pd, 1, M, K) != LBK_OK) return 0;
  return query_workspace(&pd, 1, M, K);
}

int lbk_linear_forward(const lbk_branch* branches, int n_branches, int64_t M, int64_t K, int64_t N,
                       const void* x, int x_dtype, const float* bias, void* y, int y_dtype, void* workspace,
                       size_t workspace_bytes, void* stream) {
  g_last_error[0] = '\0';
  const ProjDesc pd{branches, n_branches, N, bias, y, nullptr};
  return forward_group(&pd, 1, M, K, x, x_dtype, nullptr, y_dtype, workspace, workspace_bytes, stream);
}

int lbk_littlebit_linear(const float* input, int64_t M, const float* v2, const int32_t* v_sign, int64_t v_cols,
                         const float* mid, const int32_t* u_sign, int64_t u_cols, const float* u1,
                         int64_t out_features, float* output, void* workspace, size_t workspace_bytes,
                         void* stream) {
  lbk_branch b{};  // no tiled copy: V is read as the reference stores it
  b.v_sign = v_sign;
  b.u_sign = u_sign;
  b.v2 = v2;
  b.mid = mid;
  b.u1 = u1;
  b.rank = u_cols;
  return lbk_linear_forward(&b, 1, M, v_cols, out_features, input, LBK_F32, nullptr, output, LBK_F32, workspace,
                            workspace_bytes, stream);
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
  hipLaunchKernelGGL(pack_kernel, dim3(unsigned(blocks)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), signs,
                     rows, cols, wpr, reinterpret_cast<uint32_t*>(out));
  return check_launch("pack_kernel");
}

int64_t lbk_tiled_v_words(int64_t rank, int64_t K) {
  if (rank < 1 || K < 1) return 0;
  return ceil_div(rank, 16) * ceil_div(ceil_div(K, 32), 4) * 64;
}

int lbk_tile_v_signs(const int32_t* v_sign, int64_t rank, int64_t K, int32_t* out, void* stream) {
  g_last_error[0] = '\0';
  if (rank < 1 || K < 1 || rank > kMaxDim || K > kMaxDim)
    return set_error(LBK_ERR_ARG, "rank and K must be in [1, %lld], got %lld, %lld", (long long)kMaxDim,
                     (long long)rank, (long long)K);
  if (!v_sign || !out) return set_error(LBK_ERR_ARG, "NULL pointer");
  if (reinterpret_cast<uintptr_t>(out) & 15u) return set_error(LBK_ERR_ARG, "out must be 16-byte aligned");
  const int64_t ncell = lbk_tiled_v_words(rank, K) / 4;
  const int64_t blocks = ceil_div(ncell, kBlock) < 65536 ? ceil_div(ncell, kBlock) : 65536;
  hipLaunchKernelGGL(tile_v_kernel, dim3(unsigned(blocks)), dim3(kBlock), 0, static_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint32_t*>(v_sign), rank, ceil_div(K, 32), reinterpret_cast<u32x4*>(out));
  return check_launch("tile_v_kernel");
}

int lbk_repack_signs_to_i2(const int32_t* packed, int64_t rows, int64_t words_per_row, int64_t n_cols, uint8_t* out,
                           void* stream) {
  g_last_error[0] = '\0';
  if (rows < 0 || n_cols < 0 || words_per_row < 0) return set_error(LBK_ERR_ARG, "negative shape");
  if (words_per_row < ceil_div(n_cols, 32))
    return set_error(LBK_ERR_ARG, "n_cols (%lld) needs %lld sign words per row, packed_signs has %lld",
                     (long long)n_cols, (long long)ceil_div(n_cols, 32), (long long)words_per_row);
  const int64_t ob = ceil_div(n_cols, 4);
  if (rows == 0 || ob == 0) return LBK_OK;
  if (!packed || !out) return set_error(LBK_ERR_ARG, "NULL pointer");
  const int64_t total = rows * ceil_div(ob, 4);
  const int64_t blocks = ceil_div(total, kBlock) < 65536 ? ceil_div(total, kBlock) : 65536;
  // whole dwords when every row starts and ends on one
  const int dword_rows = (ob % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 3u) == 0) ? 1 : 0;
  hipLaunchKernelGGL(repack_i2_kernel, dim3(unsigned(blocks)), dim3(kBlock), 0, static_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint32_t*>(packed), rows, words_per_row, n_cols, ob, dword_rows, out);
  return check_launch("repack_i2_kernel");
}

size_t lbk_attention_partial_bytes(int heads, int max_seq, int head_dim) {
  if (heads < 1 || max_seq < 1 || head_dim < 1) return 0;
  const int64_t chunks = ceil_div(max_seq, kAttnChunk);
  return size_t(heads) * size_t(chunks) * size_t(head_dim + kAttnPad) * sizeof(float);
}

int lbk_attention_decode(const float* q, const float* k, const float* v, float* k_cache, float* v_cache, int heads,
                         int kv_heads, int head_dim, int max_seq, const int64_t* pos_device, int64_t pos,
                         float scale, float* partial, size_t partial_bytes, float* out, void* stream) {
  g_last_error[0] = '\0';
  if (heads < 1 || kv_heads < 1 || heads % kv_heads != 0)
    return set_error(LBK_ERR_ARG, "heads (%d) must be a positive multiple of kv_heads (%d)", heads, kv_heads);
  if (head_dim != 64 && head_dim != 128) return set_error(LBK_ERR_ARG, "head_dim must be 64 or 128, got %d", head_dim);
  if (max_seq < 1 || max_seq > (1 << 24)) return set_error(LBK_ERR_ARG, "max_seq out of range: %d", max_seq);
  if (!pos_device && (pos < 0 || pos >= max_seq))
    return set_error(LBK_ERR_ARG, "pos %lld outside [0, %d)", (long long)pos, max_seq);
  if (!q || !k || !v || !k_cache || !v_cache) return set_error(LBK_ERR_ARG, "NULL pointer");
  for (const void* ptr : {static_cast<const void*>(q), static_cast<const void*>(k), static_cast<const void*>(v),
                          static_cast<const void*>(k_cache), static_cast<const void*>(v_cache)})
    if (!aligned16(ptr)) return set_error(LBK_ERR_ARG, "q, k, v and the caches must be 16-byte aligned");
  const int chunks = int(ceil_div(max_seq, kAttnChunk));
  const size_t need = lbk_attention_partial_bytes(heads, max_seq, head_dim);
  if ((chunks > 1 || !out) && (!partial || partial_bytes < need))
    return set_error(LBK_ERR_WORKSPACE, "partial buffer of %zu bytes needed, %zu given", need, partial_bytes);
  if (!out && !aligned16(partial))
    return set_error(LBK_ERR_ARG, "partials for a consumer (out NULL) must be 16-byte aligned");
  AttnParams p;
  p.q = q;
  p.k = k;
  p.v = v;
  p.kc = k_cache;
  p.vc = v_cache;
  p.pos_ptr = pos_device;
  p.pos = pos;
  p.heads = heads;
  p.rep = heads / kv_heads;
  p.max_seq = max_seq;
  p.chunks = chunks;
  p.scale = scale;
  p.part = partial;
  p.out = out;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid{unsigned(heads), unsigned(ceil_div(chunks, kAttnThreads / 64)), 1u};
  if (head_dim == 128) hipLaunchKernelGGL(attn_decode_kernel<128>, grid, dim3(kAttnThreads), 0, s, p);
  else hipLaunchKernelGGL(attn_decode_kernel<64>, grid, dim3(kAttnThreads), 0, s, p);
  int rc = check_launch("attn_decode_kernel");
  if (rc != LBK_OK || chunks == 1 || !out) return rc;
  if (head_dim == 128) hipLaunchKernelGGL(attn_combine_kernel<128>, dim3(heads), dim3(128), 0, s, p);
  else hipLaunchKernelGGL(attn_combine_kernel<64>, dim3(heads), dim3(64), 0, s, p);
  return check_launch("attn_combine_kernel");
}

// Positions per block of attn_batch_kernel: 128 (so that the partials stay
// small next to the K and V read, and waves of up to 16 tokens walk two
// tiles, the second loading during the first; 64 measured slower at KV 1024),
// doubled while the grid would exceed 2048 blocks.
static int attn_batch_ch(int heads, int n, int64_t start) {
  int ch = 128;
  while (ch < 4096 && int64_t(heads) * ceil_div(start + n, ch) > 2048) ch *= 2;
  return ch;
}

size_t lbk_attention_batch_partial_bytes(int heads, int n, int64_t start, int head_dim) {
  if (heads < 1 || n < 1 || start < 0 || head_dim < 1) return 0;
  // (with a device start, pass max_seq - n: the grid then covers every start)
  const int64_t chunks = ceil_div(start + n, attn_batch_ch(heads, n, start));
  return size_t(heads) * size_t(chunks) * size_t(n) * size_t(head_dim + 2) * sizeof(float);
}

int lbk_attention_batch(const float* q, const float* k, const float* v, float* k_cache, float* v_cache, int n,
                        int heads, int kv_heads, int head_dim, int max_seq, const int64_t* start_device,
                        int64_t start, const uint8_t* tree_mask, float scale, float* partial, size_t partial_bytes,
                        float* out, void* stream) {
  g_last_error[0] = '\0';
  if (n < 1 || n > 64) return set_error(LBK_ERR_ARG, "n must be in [1, 64], got %d", n);
  if (heads < 1 || kv_heads < 1 || heads % kv_heads != 0)
    return set_error(LBK_ERR_ARG, "heads (%d) must be a positive multiple of kv_heads (%d)", heads, kv_heads);
  if (head_dim != 64 && head_dim != 128) return set_error(LBK_ERR_ARG, "head_dim must be 64 or 128, got %d", head_dim);
  if (max_seq < 1 || max_seq > (1 << 24)) return set_error(LBK_ERR_ARG, "max_seq out of range: %d", max_seq);
  if (n > max_seq) return set_error(LBK_ERR_ARG, "n (%d) exceeds max_seq (%d)", n, max_seq);
  if (!start_device && (start < 0 || start + n > max_seq))
    return set_error(LBK_ERR_ARG, "positions %lld .. %lld outside [0, %d)", (long long)start, (long long)(start + n - 1),
                     max_seq);
  // a device start is read at run time: size the grid for the largest one
  const int64_t sgrid = start_device ? max_seq - n : start;
  if (!q || !k || !v || !k_cache || !v_cache || !out || !partial) return set_error(LBK_ERR_ARG, "NULL pointer");
  for (const void* ptr : {static_cast<const void*>(q), static_cast<const void*>(k), static_cast<const void*>(v),
                          static_cast<const void*>(k_cache), static_cast<const void*>(v_cache)})
    if (!aligned16(ptr)) return set_error(LBK_ERR_ARG, "q, k, v and the caches must be 16-byte aligned");
  const size_t need = lbk_attention_batch_partial_bytes(heads, n, sgrid, head_dim);
  if (partial_bytes < need)
    return set_error(LBK_ERR_WORKSPACE, "partial buffer of %zu bytes needed, %zu given", need, partial_bytes);
  AttnBatchParams p;
  p.q = q;
  p.k = k;
  p.v = v;
  p.kc = k_cache;
  p.vc = v_cache;
  p.tree = tree_mask;
  p.part = partial;
  p.out = out;
  p.start_ptr = start_device;
  p.start = start;
  p.N = n;
  p.heads = heads;
  p.kvh = kv_heads;
  p.rep = heads / kv_heads;
  p.max_seq = max_seq;
  p.ch = attn_batch_ch(heads, n, sgrid);
  p.chunks = int(ceil_div(sgrid + n, p.ch));
  p.qt = n <= 16 ? 1 : n <= 32 ? 2 : 4;
  p.ps = 4 / p.qt;
  p.scale = scale;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid{unsigned(heads), unsigned(p.chunks), 1u};
  if (head_dim == 128) hipLaunchKernelGGL(attn_batch_kernel<128>, grid, dim3(kAttnThreads), 0, s, p);
  else hipLaunchKernelGGL(attn_batch_kernel<64>, grid, dim3(kAttnThreads), 0, s, p);
  int rc = check_launch("attn_batch_kernel");
  if (rc != LBK_OK) return rc;
  const dim3 cgrid{unsigned(heads), unsigned(n), 1u};
  if (head_dim == 128) hipLaunchKernelGGL(attn_batch_combine_kernel<128>, cgrid, dim3(128), 0, s, p);
  else hipLaunchKernelGGL(attn_batch_combine_kernel<64>, cgrid, dim3(64), 0, s, p);
  return check_launch("attn_batch_combine_kernel");
}

int lbk_q4_0_quantize(const float* w, int64_t rows, int64_t cols, uint8_t* qs, uint16_t* d, void* stream) {
  g_last_error[0] = '\0';
  if (rows < 0 || cols < 0 || cols % kQK != 0)
    return set_error(LBK_ERR_ARG, "rows and cols must be >= 0 with cols %% 32 == 0, got %lld x %lld",
                     (long long)rows, (long long)cols);
  const int64_t nblocks = rows * (cols / kQK);
  if (nblocks == 0) return LBK_OK;
  if (!w || !qs || !d) return set_error(LBK_ERR_ARG, "NULL pointer");
  if (!aligned16(w) || !aligned16(qs) || (reinterpret_cast<uintptr_t>(d) & 1))
    return set_error(LBK_ERR_ARG, "w and qs must be 16-byte aligned, d 2-byte aligned");
  const int64_t grid = ceil_div(nblocks, 256);
  if (grid > INT_MAX) return set_error(LBK_ERR_ARG, "weight too large");
  hipLaunchKernelGGL(q4_quantize_kernel, dim3(unsigned(grid)), dim3(256), 0, static_cast<hipStream_t>(stream), w,
                     nblocks, qs, d);
  return check_launch("q4_quantize_kernel");
}

static int head_nbl(int64_t hidden) {
  const int64_t n = ceil_div(hidden / kQK, 64);
  return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : 8;
}

static int64_t head_blocks(int64_t vocab, int64_t hidden) {
  return ceil_div(vocab, 4 * head_rows_per_wave(head_nbl(hidden)));
}

size_t lbk_lm_head_q4_workspace_bytes(int64_t vocab, int64_t hidden) {
  if (vocab < 1 || hidden < kQK) return 0;
  return align256(size_t(head_blocks(vocab, hidden)) * sizeof(uint64_t));
}

int lbk_lm_head_q4_argmax(const uint8_t* qs, const uint16_t* d, int64_t vocab, int64_t hidden, const float* x,
                          const float* norm_weight, float eps, float* logits, int64_t* token, void* workspace,
                          size_t workspace_bytes, void* stream) {
  g_last_error[0] = '\0';
  if (vocab < 1 || vocab > INT_MAX - 256)
    return set_error(LBK_ERR_ARG, "vocab out of range: %lld", (long long)vocab);
  if (hidden < kQK || hidden % kQK != 0 || hidden > 8 * 64 * kQK)
    return set_error(LBK_ERR_ARG, "hidden must be a multiple of 32 in [32, %d], got %lld", 8 * 64 * kQK,
                     (long long)hidden);
  if (!qs || !d || !x || !token) return set_error(LBK_ERR_ARG, "NULL pointer");
  if (!aligned16(qs) || !aligned16(x) || (norm_weight && !aligned16(norm_weight)) ||
      (reinterpret_cast<uintptr_t>(d) & 1))
    return set_error(LBK_ERR_ARG, "qs, x and norm_weight must be 16-byte aligned, d 2-byte aligned");
  if (norm_weight && !(eps >= 0.f)) return set_error(LBK_ERR_ARG, "eps must be >= 0");
  const size_t need = lbk_lm_head_q4_workspace_bytes(vocab, hidden);
  if (!workspace || workspace_bytes < need)
    return set_error(LBK_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  Q4HeadParams p;
  p.qs = qs;
  p.d = d;
  p.x = x;
  p.nw = norm_weight;
  p.eps = eps;
  p.V = int(vocab);
  p.H = int(hidden);
  p.logits = logits;
  p.part = static_cast<uint64_t*>(workspace);
  p.token = token;
  p.nparts = int(head_blocks(vocab, hidden));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nbl = head_nbl(hidden);
  const dim3 grid{unsigned(p.nparts)};
  if (nbl <= 1) hipLaunchKernelGGL(lm_head_q4_kernel<1>, grid, dim3(256), 0, s, p);
  else if (nbl <= 2) hipLaunchKernelGGL(lm_head_q4_kernel<2>, grid, dim3(256), 0, s, p);
  else if (nbl <= 4) hipLaunchKernelGGL(lm_head_q4_kernel<4>, grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL(lm_head_q4_kernel<8>, grid, dim3(256), 0, s, p);
  int rc = check_launch("lm_head_q4_kernel");
  if (rc != LBK_OK) return rc;
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(1), dim3(256), 0, s, p);
  return check_launch("argmax_finalize_kernel");
}

}  // extern "C"
