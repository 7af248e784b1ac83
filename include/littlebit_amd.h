/*
 * littlebit_amd.h -- C ABI of the MI355X (gfx950) LittleBitLinear forward.
 *
 *   y = sum_b  h_b * (U_b_sign . (l_b * (V_b_sign^T . (g_b * x))))  [+ bias]
 *
 * per projection, with bit-packed +-1 latent factors (one bit per sign) and
 * fp32 row / latent / column scales.  b runs over the draft ("main") branch
 * and an optional residual branch whose rank may differ from the main one.
 *
 * Conventions
 *   - Every pointer is device memory owned by the caller.  Nothing here
 *     allocates device memory or synchronises the host.
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*; NULL is the
 *     null stream) and is ordered with the caller's other work on it.
 *   - Sign words use the reference packing (LSB first, bit 1 == -1,
 *     pad bits 0 == +1); pass int32 or uint32 words, only the bits matter.
 *   - Return value 0 on success, a negative LBK_ERR_* code otherwise; the
 *     message of the last failure on the calling thread is lbk_last_error().
 *   - Workspace: caller-owned device memory, zero-filled before its first
 *     use and then kept for later calls (the library leaves its state there
 *     in a form that any later call of any shape accepts).  One workspace
 *     serves one stream; calls on different streams need different ones.
 *     Calls can be captured in a HIP graph and replayed.  A call that
 *     returns LBK_ERR_HIP may have run its first kernel and not its second;
 *     the workspace's state is then undefined: zero it again (or take a
 *     fresh zeroed one) before the next call.
 *   - Results of the MFMA path (M <= 64) are repeatable to about 1e-6
 *     relative, not bit for bit: partial sums over K meet in fp32 atomics
 *     (bit for bit under lbk_set_deterministic(1)).  The GEMM path (M > 64)
 *     is bit for bit repeatable.
 */
#ifndef LITTLEBIT_AMD_H
#define LITTLEBIT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LBK_ABI_VERSION 9

/* Element types of activations and outputs. */
#define LBK_F32 0
#define LBK_BF16 1

/* Error codes. */
#define LBK_OK 0
#define LBK_ERR_ARG (-1)       /* bad shape, null pointer, unsupported size */
#define LBK_ERR_DTYPE (-2)     /* unsupported element type */
#define LBK_ERR_WORKSPACE (-3) /* workspace missing or too small */
#define LBK_ERR_HIP (-4)       /* a HIP call or kernel launch failed */

/* One LittleBit branch of a projection with in_features K, out_features N.
 * Field names follow the runtime checkpoint keys of
 * convert_hf_to_runtime.py:46-57 (v_sign_rt, mid, u_sign_rt, u1, v2). */
typedef struct lbk_branch {
  const int32_t* v_sign; /* [rank, ceil(K/32)]  sign(V), packed along K     */
  const int32_t* u_sign; /* [N, ceil(rank/32)]  sign(U), packed along rank  */
  const float* v2;       /* [K]     column scale g                          */
  const float* mid;      /* [rank]  latent scale l = v1 * u2                */
  const float* u1;       /* [N]     row scale h                             */
  int64_t rank;          /* R >= 1                                          */
  const int32_t* v_sign_tiled; /* NULL, or v_sign tiled by lbk_tile_v_signs
                          (16-byte aligned): the decode path (M <= 64)
                          then reads V from it (whole 128-byte lines per
                          load); v_sign still serves the GEMM path         */
} lbk_branch;

/* One projection of a group call: its branches (1 or 2), out_features N,
 * optional fp32 bias [N], output y [M, N] (of the call's y_dtype) and an
 * optional fp32 residual [M, N] added to y (it may be y itself: the update
 * x += projection(...) of a decoder layer).  y may also share memory with
 * the call's input (the call then keeps its expand stage in one rank slice,
 * so that x is read before y is written).  Where the rows of a call run as
 * row chunks one after another (deterministic mode above 16 rows, or rows
 * whose latent vectors do not fit at once), the chunks run first to last,
 * or last to first, whichever reads every input row before an output row
 * overlapping it is written; a call for which neither order does returns
 * LBK_ERR_ARG. */
typedef struct lbk_projection {
  const lbk_branch* branches;
  int n_branches;
  int64_t out_features;
  const float* bias;
  void* y;
  const float* residual;
} lbk_projection;

/* What the projections of a call read (the reference's CPU decode step
 * applies these inline, patches/littlebit_cpu_optimized.cpp:1370-1438):
 *   LBK_INPUT_PLAIN     x
 *   LBK_INPUT_RMSNORM   x[m, k] / sqrt(mean_k x[m, k]^2 + rms_eps) * rms_weight[k]
 *   LBK_INPUT_SILU_MUL  x[m, k] / (1 + exp(-x[m, k])) * x1[m, k]  (x = gate, x1 = up)
 *   LBK_INPUT_ATTN_MERGE  the output of one token's attention, merged from
 *                       the per-chunk partials that lbk_attention_decode
 *                       leaves when called with out = NULL: x = those
 *                       partials (fp32, 16-byte aligned), M = 1,
 *                       K = heads * head_dim, with that call's head_dim,
 *                       max_seq and position (pos_device when not NULL, else
 *                       pos); a position outside [0, max_seq) reads as zeros.
 *                       The o projection of the decode step then needs no
 *                       separate merge launch (fused_attention_inline feeding
 *                       o_proj, patches/littlebit_cpu_optimized.cpp:1441-1510,
 *                       1736-1750). */
#define LBK_INPUT_PLAIN 0
#define LBK_INPUT_RMSNORM 1
#define LBK_INPUT_SILU_MUL 2
#define LBK_INPUT_ATTN_MERGE 3
typedef struct lbk_input {
  int kind;
  const float* rms_weight;   /* [K] fp32 (RMSNORM) */
  float rms_eps;
  const void* x1;            /* [M, K] of x_dtype (SILU_MUL) */
  int head_dim;              /* ATTN_MERGE: 64 or 128 */
  int max_seq;               /* ATTN_MERGE */
  const int64_t* pos_device; /* ATTN_MERGE: position on the device, or NULL */
  int64_t pos;               /* ATTN_MERGE: position when pos_device is NULL */
} lbk_input;

#define LBK_MAX_GROUP 4

/* ABI version (LBK_ABI_VERSION of the build). */
int lbk_abi_version(void);

/* Message of the last error on the calling thread ("" if none). */
const char* lbk_last_error(void);

/* Deterministic mode, process-wide (on != 0; returns the previous setting).
 * With it on, a decode-path call (M <= 16, and row chunks up to 64) whose
 * latent stage splits K over blocks stores each k-chunk's partial sums in
 * the workspace and the last block of each row-block to finish adds them in
 * chunk order, so outputs are the same bit for bit from run to run (off: the
 * partials meet in fp32 atomics, repeatable to about 1e-6 relative).  Both
 * modes take two launches per call.
 * The GEMM path (M > 64) is always deterministic.  Workspace sizes are
 * planned with the mode in force when queried: query (or let the Python
 * layer size its workspace) after setting it.  The reference's CPU operators
 * have no counterpart (their threads write disjoint outputs,
 * patches/littlebit_cpu_optimized.cpp:598-701); this is the race canary the
 * parity tests use. */
int lbk_set_deterministic(int on);

/* Bytes of workspace lbk_linear_forward uses for these shapes (as
 * lbk_group_workspace_bytes for one projection).
 * Returns 0 with the error set if the shapes are invalid. */
size_t lbk_linear_workspace_bytes(const lbk_branch* branches, int n_branches,
                                  int64_t M, int64_t K, int64_t N);

/* Fused LittleBitLinear forward: every branch, the branch sum and the bias.
 *   x: [M, K] of x_dtype (LBK_F32 | LBK_BF16), row-major, contiguous
 *   y: [M, N] of y_dtype (LBK_F32 | LBK_BF16), row-major, contiguous
 *   bias: [N] fp32 or NULL
 *   n_branches: 1 (draft) or 2 (draft + residual)
 * Replaces LittleBitLinear.forward / _compute_forward
 * (quantization/modules/littlebit.py:95-121), whose GPU form is two dense
 * matmuls on +-1 factors unpacked to the activation dtype. */
int lbk_linear_forward(const lbk_branch* branches, int n_branches, int64_t M,
                       int64_t K, int64_t N, const void* x, int x_dtype,
                       const float* bias, void* y, int y_dtype,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of workspace lbk_group_forward uses for these shapes (0 with the
 * error set if the shapes are invalid), for any output dtype and buffers.
 * For M > 64 this includes room for the stream-K partial tiles of stage 1;
 * a smaller workspace, down to the size without them, is accepted and runs
 * stage 1 on whole tiles. */
size_t lbk_group_workspace_bytes(const lbk_projection* projs, int n_proj,
                                 int64_t M, int64_t K);

/* Forward of up to LBK_MAX_GROUP projections that read the same x [M, K]
 * (q/k/v of a decoder layer, or gate/up), in the launches of one
 * projection: each y_p = lbk_linear_forward of projection p.  The sum of
 * all branch ranks of the group is at most 16384.  Counterpart of the
 * batched q/k/v and gate/up stages of the reference's CPU decode step
 * (patches/littlebit_cpu_optimized.cpp:1700-1723, 1777-1798). */
int lbk_group_forward(const lbk_projection* projs, int n_proj, int64_t M,
                      int64_t K, const void* x, int x_dtype, int y_dtype,
                      void* workspace, size_t workspace_bytes, void* stream);

/* lbk_group_forward with a fused input transform (input NULL = plain). */
int lbk_group_forward_ex(const lbk_projection* projs, int n_proj, int64_t M,
                         int64_t K, const void* x, int x_dtype,
                         const lbk_input* input, int y_dtype, void* workspace,
                         size_t workspace_bytes, void* stream);

/* One call of a chain: projections sharing one input (in_features K), and
 * how they read it (input NULL = plain).  Link 0 reads the chain's x like a
 * group call (any input kind).  Link j > 0 reads the outputs of link j - 1,
 * whose out_features must equal K: plain or RMSNORM (rms_weight, rms_eps)
 * read the y of link j - 1's one projection; SILU_MUL reads
 * SiLU(y_0) * y_1 of its two (gate, up; input->x1 is ignored). */
typedef struct lbk_chain_link {
  const lbk_projection* projs;
  int n_proj;
  int64_t in_features;
  const lbk_input* input;
} lbk_chain_link;

#define LBK_MAX_CHAIN 8

/* Bytes of workspace lbk_chain_forward uses for these links (0 with the
 * error set if a link is invalid); one workspace serves chains and every
 * other call on its stream. */
size_t lbk_chain_workspace_bytes(const lbk_chain_link* links, int n_links);

/* One row (M = 1, fp32 x and y) through up to LBK_MAX_CHAIN calls in
 * sequence, each writing every y of its projections (residuals, biases and
 * input kinds as in lbk_group_forward_ex): the same as calling
 * lbk_group_forward_ex link by link, in n_links + 1 launches instead of
 * 2 n_links -- each kernel between two links expands link j's rows and adds
 * their part of link j + 1's latent vector while they are still on chip.
 * The reference runs a decoder layer's projections (o, gate/up, down, and
 * the next layer's q/k/v) in one call, patches/littlebit_cpu_optimized.cpp:
 * 1627-1833 (full_forward).  Under lbk_set_deterministic(1), or for shapes
 * the joined kernel does not take (lbk_chain_fused), the links run as
 * separate calls with the same results. */
int lbk_chain_forward(const lbk_chain_link* links, int n_links, const void* x, void* workspace,
                      size_t workspace_bytes, void* stream);

/* 1 if lbk_chain_forward would run these links joined, 0 if as separate
 * calls, a negative LBK_ERR_* code if they are invalid.  No counterpart in
 * the reference (a launch-plan query). */
int lbk_chain_fused(const lbk_chain_link* links, int n_links, const void* x);

/* Bytes of the device scratch lbk_group_forward_noalloc works in. */
#define LBK_NOALLOC_SCRATCH_BYTES (8u << 20)

/* lbk_group_forward_ex without a workspace argument: it calls no hipMalloc,
 * hipFree or allocating library routine, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * it).  It has no counterpart in the reference.  Its workspace is a device
 * array of LBK_NOALLOC_SCRATCH_BYTES
 * that the library holds on each GPU it runs on until the process ends;
 * shapes whose smallest accepted workspace exceeds that return
 * LBK_ERR_WORKSPACE.  The calling thread's current device must be the
 * device of `stream`.  Every call on a GPU shares that GPU's array: calls
 * that overlap on one GPU (different streams, or threads without ordering)
 * race.  The first call on a device (and the first after a call that failed
 * with LBK_ERR_HIP) first zeroes the array with a kernel on `stream`; when
 * `stream` is being captured, that kernel is part of the graph (it runs in
 * every replay) and the next eager call zeroes the array again. */
int lbk_group_forward_noalloc(const lbk_projection* projs, int n_proj, int64_t M, int64_t K, const void* x,
                              int x_dtype, const lbk_input* input, int y_dtype, void* stream);

/* One-branch form with the argument list of the reference operator
 * littlebit_cpu_ops::littlebit_linear (patches/littlebit_cpu_optimized.cpp:
 * 598-701, schema at :2324-2329): input [M, v_cols] fp32, v2 [1, v_cols],
 * v_sign [R, ceil(v_cols/32)], mid [1, R], u_sign [N, ceil(u_cols/32)],
 * u1 [1, N], u_cols == R; output [M, N] fp32.  The reference quantises the
 * activations to int8 at both stages; this computes in fp32 throughout. */
int lbk_littlebit_linear(const float* input, int64_t M, const float* v2,
                         const int32_t* v_sign, int64_t v_cols,
                         const float* mid, const int32_t* u_sign,
                         int64_t u_cols, const float* u1, int64_t out_features,
                         float* output, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Decode attention of one query token (the draft step's attention), fp32,
 * kv_heads dividing heads, no rotary embedding, head_dim 64 or 128:
 *   out[h] = sum_t softmax_t(scale * q[h] . K[h/r][t]) V[h/r][t], t = 0..pos
 * where K/V[.][pos] are the new k, v [kv_heads * head_dim], which are also
 * stored into k_cache / v_cache [kv_heads][max_seq][head_dim].  pos is read
 * from pos_device when it is not NULL (so a captured graph follows a
 * position the device advances), else taken from pos.  partial: scratch of
 * lbk_attention_partial_bytes() (needed when max_seq > 16 or out is NULL).
 * A position outside [0, max_seq) stores nothing and yields zeros.  With
 * out = NULL the call stops at the per-chunk partials (partial 16-byte
 * aligned), which a projection reads with LBK_INPUT_ATTN_MERGE.
 * Replaces fused_attention_inline (patches/littlebit_cpu_optimized.cpp:
 * 1441-1510) and the per-token attention of cpu_draft_model.py:371-383. */
size_t lbk_attention_partial_bytes(int heads, int max_seq, int head_dim);
int lbk_attention_decode(const float* q, const float* k, const float* v,
                         float* k_cache, float* v_cache, int heads,
                         int kv_heads, int head_dim, int max_seq,
                         const int64_t* pos_device, int64_t pos, float scale,
                         float* partial, size_t partial_bytes, float* out,
                         void* stream);

/* Attention of n new tokens (1 <= n <= 64) at positions start .. start+n-1,
 * fp32, kv_heads dividing heads, no rotary embedding, head_dim 64 or 128:
 *   out[i][h] = sum_t softmax_t(scale * q[i][h] . K[h/r][t]) V[h/r][t]
 * over t < start (the cache) and the new tokens t = start + j that token i
 * sees: j <= i (causal, tree_mask NULL), or tree_mask[i * n + j] != 0
 * (uint8 [n][n]).  q [n][heads * head_dim], k, v [n][kv_heads * head_dim]
 * (the new keys and values, also stored into k_cache / v_cache
 * [kv_heads][max_seq][head_dim]); q, k, v and the caches 16-byte aligned;
 * out [n][heads * head_dim].  start is read from start_device when that is
 * not NULL (a captured graph then follows a position the device advances;
 * a start with positions outside [0, max_seq) stores nothing and yields
 * zeros).  partial: scratch of lbk_attention_batch_partial_bytes(heads, n,
 * start, head_dim), with start = max_seq - n for a device start.  Replaces the attention of the
 * batched decode step (patches/littlebit_cpu_optimized.cpp:1846-2079) and the
 * tree-masked attention of tree verification (tree_utils.py:72-214). */
size_t lbk_attention_batch_partial_bytes(int heads, int n, int64_t start, int head_dim);
int lbk_attention_batch(const float* q, const float* k, const float* v,
                        float* k_cache, float* v_cache, int n, int heads,
                        int kv_heads, int head_dim, int max_seq,
                        const int64_t* start_device, int64_t start,
                        const uint8_t* tree_mask, float scale, float* partial,
                        size_t partial_bytes, float* out, void* stream);

/* Expand packed signs to int8 {-1,+1}: out [rows, cols].
 * Replaces binary_unpacker (quantization/utils/binary_packer.py:54-97). */
int lbk_unpack_signs(const int32_t* packed, int64_t rows, int64_t cols,
                     int8_t* out, void* stream);

/* Pack int8 signs to words: out [rows, ceil(cols/32)]; s < 0 -> bit 1, else
 * bit 0, pad bits 0.  Same words as binary_packer
 * (quantization/utils/binary_packer.py:5-51) for inputs in {-1, +1}. */
int lbk_pack_signs(const int8_t* signs, int64_t rows, int64_t cols,
                   int32_t* out, void* stream);

/* Words of V's tiled copy for lbk_branch.v_sign_tiled:
 * ceil(rank/16) * ceil(ceil(K/32)/4) * 64 (0 for rank or K < 1).  No
 * counterpart in the reference (a GPU load layout). */
int64_t lbk_tiled_v_words(int64_t rank, int64_t K);

/* Tile V's sign words [rank, ceil(K/32)] into out (lbk_tiled_v_words
 * int32, 16-byte aligned): [ceil(rank/16)][ceil(KW/4)][16 rows][4 words],
 * word w of row r at ((r/16 * ceil(KW/4) + w/4) * 16 + r%16) * 4 + w%4,
 * zero past rank and past KW = ceil(K/32).  Done once at load time, like the
 * reference's repack of its sign words for its own kernel
 * (cpu_draft_model.py:247-250). */
int lbk_tile_v_signs(const int32_t* v_sign, int64_t rank, int64_t K,
                     int32_t* out, void* stream);

/* Sign words [rows, words_per_row] -> the 2-bit layout of the reference's CPU
 * runtime, out [rows, ceil(n_cols/4)] uint8, byte for byte what
 * repack_signs_to_i2 (patches/littlebit_cpu_optimized.cpp:712-764, schema at
 * :2340; called by cpu_draft_model.py:247-250) writes: column
 * c = 128 b + 32 g + p is the field at bit shift 6 - 2 g of byte 32 b + p,
 * 2 for +1 and 0 for -1.  As in the reference, a column whose byte index is
 * >= ceil(n_cols/4) is dropped (the last block of a row when n_cols % 128 != 0)
 * and fields no column fills are 0.  words_per_row must be at least
 * ceil(n_cols/32) (LBK_ERR_ARG otherwise; the reference reads past the row). */
int lbk_repack_signs_to_i2(const int32_t* packed, int64_t rows,
                           int64_t words_per_row, int64_t n_cols,
                           uint8_t* out, void* stream);

/* Q4_0 quantisation of an lm_head weight w [rows][cols] fp32 (cols % 32 == 0),
 * as the reference's quantize_lm_head_q4 (patches/littlebit_cpu_optimized.cpp:
 * 2129-2149, 2225-2251) computes it, bit for bit: per block of 32 the fp16
 * scale d = m / -8 (m the first value of largest magnitude; fp16 by
 * truncation, :2119-2127) and nibbles q = min(15, int(x / d + 8.5)).  Stored
 * as two planes instead of the reference's 18-byte blocks: qs [rows][cols/2]
 * (byte j of a block holds value j in its low nibble and value j + 16 in its
 * high nibble, as the reference packs them; 16-byte aligned) and d
 * [rows][cols/32] (fp16 bits). */
int lbk_q4_0_quantize(const float* w, int64_t rows, int64_t cols, uint8_t* qs,
                      uint16_t* d, void* stream);

/* The tail of the reference's generate_token (patch:2254-2317): the final
 * hidden state x [hidden] -- RMS-normed first with norm_weight and eps when
 * norm_weight is not NULL (rms_norm_inline, patch:1370-1405) -- quantised to
 * Q8_0 (d = amax / 127, q = round(x / d); :2152-2165), the Q4_0 x Q8_0
 * logits of the vocab rows (:2168-2222; also written to logits [vocab] when
 * that is not NULL), and the first index of the largest logit written to
 * *token (device int64).  hidden % 32 == 0, hidden <= 16384; qs, x and
 * norm_weight 16-byte aligned.  workspace: lbk_lm_head_q4_workspace_bytes(). */
size_t lbk_lm_head_q4_workspace_bytes(int64_t vocab, int64_t hidden);
int lbk_lm_head_q4_argmax(const uint8_t* qs, const uint16_t* d, int64_t vocab,
                          int64_t hidden, const float* x,
                          const float* norm_weight, float eps, float* logits,
                          int64_t* token, void* workspace,
                          size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LITTLEBIT_AMD_H */
