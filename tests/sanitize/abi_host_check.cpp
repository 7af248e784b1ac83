// Host-side check of the C ABI's validation and planning code, built with
// AddressSanitizer and UndefinedBehaviorSanitizer on the host pass only
// (tests/test_host_sanitizers.py).  It makes no device call: workspace
// queries (which run the whole launch planning: path choice, row chunks,
// expand shapes, stream-K sizing) over a grid of shapes, and every argument
// error the entry points return before a launch.  Factor pointers are fake
// aligned addresses that the host code never dereferences.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "littlebit_amd.h"

static int failures = 0;
#define EXPECT(cond, ...)                         \
  do {                                            \
    if (!(cond)) {                                \
      std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
      std::printf(__VA_ARGS__);                   \
      std::printf(" [%s]\n", lbk_last_error());   \
      ++failures;                                 \
    }                                             \
  } while (0)

static const void* fake(uintptr_t i) { return reinterpret_cast<const void*>(uintptr_t(0x100000) * (i + 1)); }

static lbk_branch branch(int64_t rank, uintptr_t tag) {
  lbk_branch b{};
  b.v_sign = static_cast<const int32_t*>(fake(tag));
  b.u_sign = static_cast<const int32_t*>(fake(tag + 1));
  b.v2 = static_cast<const float*>(fake(tag + 2));
  b.mid = static_cast<const float*>(fake(tag + 3));
  b.u1 = static_cast<const float*>(fake(tag + 4));
  b.rank = rank;
  return b;
}

int main() {
  EXPECT(lbk_abi_version() == LBK_ABI_VERSION, "abi version");
  // ---- workspace queries over shapes: planning for every path
  const int64_t Ms[] = {0, 1, 2, 3, 7, 8, 9, 15, 16, 17, 31, 33, 48, 63, 64, 65, 100, 128, 129, 300, 1000, 2048, 4096};
  const int64_t Ks[] = {1, 31, 32, 33, 64, 70, 1000, 4096, 4160, 11008, 14336};
  const int64_t ranks[][2] = {{1, 0}, {31, 0}, {205, 0}, {205, 1843}, {298, 2686}, {318, 2867}, {4000, 4000}, {32, 33}};
  const int64_t Ns[] = {1, 33, 300, 1024, 4096, 14336};
  size_t queries = 0;
  for (int64_t K : Ks)
    for (auto& rk : ranks)
      for (int64_t N : Ns)
        for (int nproj = 1; nproj <= LBK_MAX_GROUP; ++nproj) {
          std::vector<lbk_branch> br;
          for (int q = 0; q < nproj; ++q) {
            br.push_back(branch(rk[0], 10 * q));
            if (rk[1]) br.push_back(branch(rk[1], 10 * q + 5));
          }
          const int nb = rk[1] ? 2 : 1;
          std::vector<lbk_projection> pj(nproj);
          for (int q = 0; q < nproj; ++q)
            pj[q] = lbk_projection{br.data() + q * nb, nb, N, nullptr, const_cast<void*>(fake(99)), nullptr};
          const int64_t rsum = nproj * (rk[0] + rk[1]);
          for (int64_t M : Ms) {
            const size_t g = lbk_group_workspace_bytes(pj.data(), nproj, M, K);
            ++queries;
            if (rsum <= 16384) {
              EXPECT(g > 0, "group workspace M=%lld K=%lld N=%lld nproj=%d", (long long)M, (long long)K, (long long)N,
                     nproj);
            } else {
              EXPECT(g == 0 && std::strlen(lbk_last_error()) > 0, "rank sum %lld accepted", (long long)rsum);
            }
            if (nproj == 1) {
              const size_t l = lbk_linear_workspace_bytes(br.data(), nb, M, K, N);
              EXPECT(l > 0, "linear workspace");
              EXPECT(l == g, "linear (%zu) and one-projection group (%zu) workspaces differ", l, g);
            }
          }
        }
  std::printf("%zu workspace queries\n", queries);
  // deterministic mode adds the k-chunk partials to decode-path workspaces
  EXPECT(lbk_set_deterministic(1) == 0, "deterministic mode starts off");
  for (int64_t M : {int64_t(1), int64_t(8), int64_t(16), int64_t(33), int64_t(64), int64_t(100)}) {
    lbk_branch bd[2] = {branch(298, 0), branch(2686, 5)};
    lbk_projection pd{bd, 2, 11008, nullptr, const_cast<void*>(fake(99)), nullptr};
    const size_t on = lbk_group_workspace_bytes(&pd, 1, M, 4096);
    lbk_set_deterministic(0);
    const size_t off = lbk_group_workspace_bytes(&pd, 1, M, 4096);
    lbk_set_deterministic(1);
    EXPECT(on >= off && off > 0, "deterministic workspace M=%lld: %zu vs %zu", (long long)M, on, off);
  }
  EXPECT(lbk_set_deterministic(0) == 1, "deterministic mode was on");

  // ---- argument errors (each returns before any launch)
  lbk_branch b2[2] = {branch(205, 0), branch(1843, 5)};
  lbk_projection p1{b2, 2, 4096, nullptr, const_cast<void*>(fake(99)), nullptr};
  float* xf = const_cast<float*>(static_cast<const float*>(fake(50)));
  void* ws = const_cast<void*>(fake(60));
  const size_t wsz = lbk_group_workspace_bytes(&p1, 1, 8, 4096);
  EXPECT(lbk_group_forward(nullptr, 1, 8, 4096, xf, LBK_F32, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG, "NULL projs");
  EXPECT(lbk_group_forward(&p1, 0, 8, 4096, xf, LBK_F32, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG, "n_proj 0");
  EXPECT(lbk_group_forward(&p1, LBK_MAX_GROUP + 1, 8, 4096, xf, LBK_F32, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG,
         "n_proj too large");
  EXPECT(lbk_group_forward(&p1, 1, -1, 4096, xf, LBK_F32, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG, "M < 0");
  EXPECT(lbk_group_forward(&p1, 1, 8, 0, xf, LBK_F32, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG, "K = 0");
  EXPECT(lbk_group_forward(&p1, 1, 8, int64_t(1) << 40, xf, LBK_F32, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG,
         "K huge");
  EXPECT(lbk_group_forward(&p1, 1, 8, 4096, nullptr, LBK_F32, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG, "NULL x");
  EXPECT(lbk_group_forward(&p1, 1, 8, 4096, xf, 7, LBK_F32, ws, wsz, nullptr) == LBK_ERR_DTYPE, "x dtype");
  EXPECT(lbk_group_forward(&p1, 1, 8, 4096, xf, LBK_F32, 9, ws, wsz, nullptr) == LBK_ERR_DTYPE, "y dtype");
  EXPECT(lbk_group_forward(&p1, 1, 8, 4096, xf, LBK_F32, LBK_F32, nullptr, wsz, nullptr) == LBK_ERR_WORKSPACE,
         "NULL workspace");
  EXPECT(lbk_group_forward(&p1, 1, 8, 4096, xf, LBK_F32, LBK_F32, ws, wsz - 1, nullptr) == LBK_ERR_WORKSPACE,
         "small workspace");
  // the mode is read once per call, when the call is planned: a workspace
  // sized with deterministic mode off is refused, before any launch, by a
  // call made after the mode was turned on (side-by-side row chunks off,
  // sequential chunks with k-chunk partials on)
  for (int64_t M : {int64_t(1), int64_t(8), int64_t(33), int64_t(48)}) {
    const size_t off = lbk_group_workspace_bytes(&p1, 1, M, 4096);
    lbk_set_deterministic(1);
    const size_t on = lbk_group_workspace_bytes(&p1, 1, M, 4096);
    EXPECT(on > off && off > 0, "deterministic workspace M=%lld: %zu vs %zu", (long long)M, on, off);
    EXPECT(lbk_group_forward(&p1, 1, M, 4096, xf, LBK_F32, LBK_F32, ws, off, nullptr) == LBK_ERR_WORKSPACE,
           "mode turned on after the query, M=%lld", (long long)M);
    lbk_set_deterministic(0);
  }
  {
    lbk_projection p = p1;
    p.y = nullptr;
    EXPECT(lbk_group_forward(&p, 1, 8, 4096, xf, LBK_F32, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG, "NULL y");
    p = p1;
    p.n_branches = 3;
    EXPECT(lbk_group_workspace_bytes(&p, 1, 8, 4096) == 0, "3 branches");
    p = p1;
    p.out_features = 0;
    EXPECT(lbk_group_workspace_bytes(&p, 1, 8, 4096) == 0, "N = 0");
    p = p1;
    p.branches = nullptr;
    EXPECT(lbk_group_workspace_bytes(&p, 1, 8, 4096) == 0, "NULL branches");
    lbk_branch bad[2] = {b2[0], b2[1]};
    bad[1].rank = 0;
    p = p1;
    p.branches = bad;
    EXPECT(lbk_group_workspace_bytes(&p, 1, 8, 4096) == 0, "rank 0");
    bad[1] = b2[1];
    bad[1].mid = nullptr;
    EXPECT(lbk_group_workspace_bytes(&p, 1, 8, 4096) == 0, "NULL mid");
  }
  // fused inputs
  {
    lbk_input in{};
    in.kind = 9;
    EXPECT(lbk_group_forward_ex(&p1, 1, 8, 4096, xf, LBK_F32, &in, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG,
           "unknown input kind");
    in.kind = LBK_INPUT_RMSNORM;
    in.rms_weight = nullptr;
    EXPECT(lbk_group_forward_ex(&p1, 1, 8, 4096, xf, LBK_F32, &in, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG,
           "RMSNORM without weight");
    in.kind = LBK_INPUT_SILU_MUL;
    in.x1 = nullptr;
    EXPECT(lbk_group_forward_ex(&p1, 1, 8, 4096, xf, LBK_F32, &in, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG,
           "SILU_MUL without x1");
    in.kind = LBK_INPUT_ATTN_MERGE;
    in.head_dim = 96;
    in.max_seq = 512;
    EXPECT(lbk_group_forward_ex(&p1, 1, 1, 4096, xf, LBK_F32, &in, LBK_F32, ws, wsz, nullptr) == LBK_ERR_ARG,
           "ATTN_MERGE head_dim");
  }
  // allocation-free entry: shapes beyond its scratch are refused before any device call
  {
    lbk_branch big[2] = {branch(4000, 0), branch(4000, 5)};
    lbk_projection pb{big, 2, 14336, nullptr, const_cast<void*>(fake(99)), nullptr};
    EXPECT(lbk_group_forward_noalloc(&pb, 1, 4096, 14336, xf, LBK_F32, nullptr, LBK_F32, nullptr) ==
               LBK_ERR_WORKSPACE,
           "noalloc refuses a large shape");
  }
  // reference-form operator
  EXPECT(lbk_littlebit_linear(xf, 4, xf, static_cast<const int32_t*>(fake(1)), 4096, xf,
                              static_cast<const int32_t*>(fake(2)), 100, xf, 0, xf, ws, wsz, nullptr) == LBK_ERR_ARG,
         "out_features 0");
  EXPECT(lbk_littlebit_linear(xf, 4, xf, static_cast<const int32_t*>(fake(1)), 4096, xf,
                              static_cast<const int32_t*>(fake(2)), 0, xf, 4096, xf, ws, wsz, nullptr) == LBK_ERR_ARG,
         "u_cols (the rank) 0");
  // signs, attention, lm head
  EXPECT(lbk_unpack_signs(static_cast<const int32_t*>(fake(1)), -1, 5, reinterpret_cast<int8_t*>(ws), nullptr) ==
             LBK_ERR_ARG,
         "unpack negative rows");
  EXPECT(lbk_pack_signs(nullptr, 3, 5, reinterpret_cast<int32_t*>(ws), nullptr) == LBK_ERR_ARG, "pack NULL");
  EXPECT(lbk_attention_partial_bytes(32, 1024, 128) > 0, "attention partial bytes");
  EXPECT(lbk_attention_batch_partial_bytes(32, 33, 1024, 128) > 0, "batch partial bytes");
  EXPECT(lbk_attention_decode(xf, xf, xf, xf, xf, 32, 5, 128, 512, nullptr, 0, 1.f, xf, 1 << 20, xf, nullptr) ==
             LBK_ERR_ARG,
         "heads not a multiple of kv_heads");
  EXPECT(lbk_attention_batch(xf, xf, xf, xf, xf, 65, 32, 8, 128, 1024, nullptr, 0, nullptr, 1.f, xf, 1 << 20, xf,
                             nullptr) == LBK_ERR_ARG,
         "batch n > 64");
  EXPECT(lbk_q4_0_quantize(xf, 4, 33, static_cast<uint8_t*>(ws), static_cast<uint16_t*>(ws), nullptr) == LBK_ERR_ARG,
         "q4 cols % 32");
  EXPECT(lbk_lm_head_q4_workspace_bytes(32000, 4096) > 0, "lm head workspace");
  EXPECT(lbk_lm_head_q4_argmax(static_cast<const uint8_t*>(ws), static_cast<const uint16_t*>(ws), 32000, 4100, xf,
                               nullptr, 1e-6f, nullptr, static_cast<int64_t*>(ws), ws, 1 << 20, nullptr) == LBK_ERR_ARG,
         "lm head hidden % 32");

  // ---- chains (lbk_chain_*): a draft decoder layer o -> gate/up -> down ->
  // next q/k/v, its planning and every error returned before a launch
  {
    auto tiled = [](int64_t rank, uintptr_t tag) {
      lbk_branch b = branch(rank, tag);
      b.v_sign_tiled = static_cast<const int32_t*>(fake(tag + 6));
      return b;
    };
    lbk_branch bo = tiled(205, 100), bg = tiled(298, 110), bu = tiled(298, 120), bd = tiled(298, 130);
    lbk_branch bq = tiled(205, 140), bk = tiled(205, 150), bv = tiled(205, 160);
    void* X = const_cast<void*>(fake(200));
    void* G = const_cast<void*>(fake(210));
    void* U = const_cast<void*>(fake(220));
    void* Q = const_cast<void*>(fake(230));
    void* Kk = const_cast<void*>(fake(240));
    void* V = const_cast<void*>(fake(250));
    const float* Xr = static_cast<const float*>(X);
    lbk_projection po{&bo, 1, 4096, nullptr, X, Xr};
    lbk_projection pgu[2] = {{&bg, 1, 11008, nullptr, G, nullptr}, {&bu, 1, 11008, nullptr, U, nullptr}};
    lbk_projection pdn{&bd, 1, 4096, nullptr, X, Xr};
    lbk_projection pqkv[3] = {{&bq, 1, 4096, nullptr, Q, nullptr}, {&bk, 1, 4096, nullptr, Kk, nullptr},
                              {&bv, 1, 4096, nullptr, V, nullptr}};
    lbk_input plain{};
    plain.kind = LBK_INPUT_PLAIN;
    lbk_input rms2{}, rms1{}, silu{};
    rms2.kind = rms1.kind = LBK_INPUT_RMSNORM;
    rms2.rms_weight = static_cast<const float*>(fake(400));
    rms1.rms_weight = static_cast<const float*>(fake(410));
    rms2.rms_eps = rms1.rms_eps = 1e-5f;
    silu.kind = LBK_INPUT_SILU_MUL;
    lbk_chain_link layer[4] = {{&po, 1, 4096, &plain}, {pgu, 2, 4096, &rms2}, {&pdn, 1, 11008, &silu},
                               {pqkv, 3, 4096, &rms1}};
    const void* x0 = fake(300);
    const size_t cw = lbk_chain_workspace_bytes(layer, 4);
    EXPECT(cw > 0, "chain workspace");
    EXPECT(cw >= lbk_group_workspace_bytes(pgu, 2, 1, 4096), "chain workspace below a link's");
    EXPECT(lbk_chain_fused(layer, 4, x0) == 1, "the draft layer's chain runs joined");
    EXPECT(lbk_chain_fused(layer, 1, x0) == 0, "one link runs as a call");
    {
      lbk_input silu0 = silu;  // the first link's SiLU * up reads the caller's x and x1
      silu0.x1 = fake(310);
      lbk_chain_link tail[2] = {{&pdn, 1, 11008, &silu0}, layer[3]};
      EXPECT(lbk_chain_fused(tail, 2, x0) == 1, "down -> q/k/v with SiLU * up of the caller's x, x1");
      lbk_chain_link nox1[2] = {{&pdn, 1, 11008, &silu}, layer[3]};
      EXPECT(lbk_chain_fused(nox1, 2, x0) == LBK_ERR_ARG, "first link's SiLU * up without x1");
    }
    lbk_set_deterministic(1);
    EXPECT(lbk_chain_fused(layer, 4, x0) == 0, "deterministic mode runs the links apart");
    lbk_set_deterministic(0);
    // without V's tiled copy the links run apart
    lbk_branch bd_plain = bd;
    bd_plain.v_sign_tiled = nullptr;
    lbk_projection pdn_plain{&bd_plain, 1, 4096, nullptr, X, Xr};
    lbk_chain_link untiled[4] = {layer[0], layer[1], {&pdn_plain, 1, 11008, &silu}, layer[3]};
    EXPECT(lbk_chain_fused(untiled, 4, x0) == 0, "an untiled V runs apart");
    // the longest chain: plain links alternating 4096 -> 4096
    {
      lbk_chain_link eight[LBK_MAX_CHAIN];
      for (int j = 0; j < LBK_MAX_CHAIN; ++j) eight[j] = {&po, 1, 4096, &plain};
      EXPECT(lbk_chain_workspace_bytes(eight, LBK_MAX_CHAIN) > 0, "eight links");
      EXPECT(lbk_chain_fused(eight, LBK_MAX_CHAIN, x0) == 1, "eight links run joined");
      lbk_chain_link nine[LBK_MAX_CHAIN + 1];
      for (int j = 0; j <= LBK_MAX_CHAIN; ++j) nine[j] = {&po, 1, 4096, &plain};
      EXPECT(lbk_chain_forward(nine, LBK_MAX_CHAIN + 1, x0, ws, 1u << 30, nullptr) == LBK_ERR_ARG, "nine links");
    }
    EXPECT(lbk_chain_forward(nullptr, 2, x0, ws, cw, nullptr) == LBK_ERR_ARG, "NULL links");
    EXPECT(lbk_chain_forward(layer, 0, x0, ws, cw, nullptr) == LBK_ERR_ARG, "no links");
    EXPECT(lbk_chain_forward(layer, 4, x0, ws, cw - 1, nullptr) == LBK_ERR_WORKSPACE, "small chain workspace");
    EXPECT(lbk_chain_forward(layer, 4, x0, nullptr, cw, nullptr) == LBK_ERR_WORKSPACE, "NULL chain workspace");
    {
      lbk_chain_link bad[2] = {{&po, 1, 4096, &plain}, {&pdn, 1, 11008, &silu}};  // SiLU * up after one projection
      EXPECT(lbk_chain_forward(bad, 2, x0, ws, 1u << 30, nullptr) == LBK_ERR_ARG, "SiLU after one projection");
      EXPECT(std::strstr(lbk_last_error(), "link 1") != nullptr, "error names the link");
    }
    {
      lbk_chain_link bad[2] = {{pgu, 2, 4096, &rms2}, {&po, 1, 4096, &plain}};  // plain after two projections
      EXPECT(lbk_chain_forward(bad, 2, x0, ws, 1u << 30, nullptr) == LBK_ERR_ARG, "plain after two projections");
    }
    {
      lbk_chain_link bad[2] = {{&po, 1, 4096, &plain}, {&pdn, 1, 11008, &plain}};  // K 11008 after N 4096
      EXPECT(lbk_chain_forward(bad, 2, x0, ws, 1u << 30, nullptr) == LBK_ERR_ARG, "in_features mismatch");
    }
    {
      lbk_input merge{};
      merge.kind = LBK_INPUT_ATTN_MERGE;
      merge.head_dim = 128;
      merge.max_seq = 512;
      lbk_chain_link bad[2] = {{&po, 1, 4096, &plain}, {&po, 1, 4096, &merge}};  // a merge input mid-chain
      EXPECT(lbk_chain_forward(bad, 2, x0, ws, 1u << 30, nullptr) == LBK_ERR_ARG, "attention merge mid-chain");
    }
    {
      lbk_chain_link bad[1] = {{&po, 0, 4096, &plain}};
      EXPECT(lbk_chain_forward(bad, 1, x0, ws, 1u << 30, nullptr) == LBK_ERR_ARG, "link without projections");
    }
  }
  std::printf("%s (%d failures)\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
