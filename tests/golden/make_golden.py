"""Write the golden fixtures under tests/golden/.

Nothing here imports the oracle or the package: expected values come from
first principles so that they can pin both.

pack_vectors.json
    Hand-built sign rows and the int32 words the reference packer
    (quantization/utils/binary_packer.py:36-50) must produce: LSB first,
    bit 1 == -1, pad with +1 (bit 0), int32 two's complement.

forward_small.npz
    Small LittleBit projections (ragged K, R, N; one and two branches with
    different ranks; bias) with the output of
        y[m, n] = bias[n] + sum_b h_b[n] * sum_r sU_b[n, r] * l_b[r]
                            * sum_k sV_b[r, k] * g_b[k] * x[m, k]
    evaluated term by term with Python integers for the bits and math.fsum
    (correctly rounded sums) for the arithmetic.

synthetic_digests.json
    SHA-256 of the arrays the seeded generator draws for the single-layer
    benchmark configurations 0 and 1 (numpy PCG64, seed 1000 + index), so that a numpy change that
    alters the stream is caught.

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import math
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


# ---------------------------------------------------------------------------
# pack vectors
# ---------------------------------------------------------------------------
def word_from_signs(signs32):
    """Bits of one word from 32 signs, as an int32 value."""
    v = 0
    for j, s in enumerate(signs32):
        if s == -1:
            v |= 1 << j
    return v - (1 << 32) if v >= 1 << 31 else v


def pack_row(signs):
    cols = len(signs)
    wpr = (cols + 31) // 32
    padded = list(signs) + [1] * (wpr * 32 - cols)
    return [word_from_signs(padded[32 * w:32 * w + 32]) for w in range(wpr)]


def pack_vectors():
    cases = []

    def add(name, rows):
        cases.append({"name": name, "cols": len(rows[0]), "signs": rows, "words": [pack_row(r) for r in rows]})

    only31 = [1] * 32
    only31[31] = -1
    add("bit31_only", [only31])                          # -> -2147483648
    add("all_minus_32", [[-1] * 32])                     # -> -1 (0xFFFFFFFF)
    add("all_plus_32", [[1] * 32])                       # -> 0
    add("alternating_32", [[-1 if j % 2 == 0 else 1 for j in range(32)]])   # 0x55555555
    add("cols_1_2_neg", [[1, -1, -1, 1] + [1] * 28])     # -> 6
    add("ragged_70_all_minus", [[-1] * 70])              # -> [-1, -1, 63]
    add("ragged_70_all_plus", [[1] * 70])                # -> [0, 0, 0]
    add("ragged_5", [[-1, 1, 1, 1, -1]])                 # -> 17
    rng = np.random.Generator(np.random.PCG64(7))
    rows = (1 - 2 * rng.integers(0, 2, size=(3, 77))).astype(int).tolist()
    add("random_3x77", rows)
    # hand-checked expectations for the simple cases
    expect = {
        "bit31_only": [[-2147483648]],
        "all_minus_32": [[-1]],
        "all_plus_32": [[0]],
        "alternating_32": [[0x55555555]],
        "cols_1_2_neg": [[6]],
        "ragged_70_all_minus": [[-1, -1, 63]],
        "ragged_70_all_plus": [[0, 0, 0]],
        "ragged_5": [[17]],
    }
    for c in cases:
        if c["name"] in expect:
            assert c["words"] == expect[c["name"]], (c["name"], c["words"])
    return cases


# ---------------------------------------------------------------------------
# forward fixtures
# ---------------------------------------------------------------------------
def rand_words(rng, rows, cols):
    wpr = (cols + 31) // 32
    w = rng.integers(0, 2**32, size=(rows, wpr), dtype=np.uint64)
    tail = cols - 32 * (wpr - 1)
    if tail < 32:
        w[:, -1] &= (1 << tail) - 1
    return w.astype(np.uint32).view(np.int32)


def bit_sign(words_u32_row, col):
    word = int(words_u32_row[col // 32])
    return -1 if (word >> (col % 32)) & 1 else 1


def brute_force(x, branches, bias, K, N):
    M = x.shape[0]
    y = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        xm = [float(v) for v in x[m]]
        terms_n = [[] for _ in range(N)]
        for br in branches:
            R = br["R"]
            vw = br["v_sign"].view(np.uint32)
            uw = br["u_sign"].view(np.uint32)
            g, l, h = br["g"], br["l"], br["h"]
            t = []
            for r in range(R):
                s = math.fsum(bit_sign(vw[r], k) * float(g[k]) * xm[k] for k in range(K))
                t.append(float(l[r]) * s)
            for n in range(N):
                s = math.fsum(bit_sign(uw[n], r) * t[r] for r in range(R))
                terms_n[n].append(float(h[n]) * s)
        for n in range(N):
            if bias is not None:
                terms_n[n].append(float(bias[n]))
            y[m, n] = math.fsum(terms_n[n])
    return y


def scales(rng, n):
    return (np.abs(rng.standard_normal(n)) + 0.05).astype(np.float32)


FORWARD_CASES = [
    # name, seed, M, K, N, ranks, bias
    ("tiny_1branch", 11, 1, 32, 32, [1], False),
    ("ragged_1branch", 12, 3, 70, 45, [37], False),
    ("ragged_2branch", 13, 2, 70, 45, [9, 33], True),
    ("wide_2branch", 14, 4, 96, 64, [40, 65], False),
    ("m5_odd", 15, 5, 33, 31, [31, 1], True),
]


def forward_fixtures():
    out = {}
    for name, seed, M, K, N, ranks, with_bias in FORWARD_CASES:
        rng = np.random.Generator(np.random.PCG64(seed))
        x = rng.standard_normal((M, K)).astype(np.float32)
        branches = []
        for R in ranks:
            v = rand_words(rng, R, K)
            u = rand_words(rng, N, R)
            branches.append({"R": R, "v_sign": v, "u_sign": u, "g": scales(rng, K), "l": scales(rng, R),
                             "h": scales(rng, N)})
        bias = rng.standard_normal(N).astype(np.float32) if with_bias else None
        y = brute_force(x, branches, bias, K, N)
        out[f"{name}/meta"] = np.array([M, K, N, len(ranks), int(with_bias)], dtype=np.int64)
        out[f"{name}/x"] = x
        for i, b in enumerate(branches):
            for key in ("v_sign", "u_sign", "g", "l", "h"):
                out[f"{name}/b{i}/{key}"] = b[key]
        if bias is not None:
            out[f"{name}/bias"] = bias
        out[f"{name}/y"] = y
    return out


# ---------------------------------------------------------------------------
# synthetic-stream digests (mirrors littlebit_amd.synthetic's draw order)
# ---------------------------------------------------------------------------
def _pack_bits_le(signs):
    rows, cols = signs.shape
    wpr = (cols + 31) // 32
    bits = np.zeros((rows, wpr * 32), dtype=np.uint8)
    bits[:, :cols] = signs < 0
    return np.packbits(bits, axis=1, bitorder="little").view("<u4").view(np.int32).reshape(rows, wpr)


def synthetic_digests():
    def sha(a):
        return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()

    res = {}
    for cfg, M, ranks in ((0, 1, [205]), (1, 8, [205, 1843])):
        rng = np.random.Generator(np.random.PCG64(1000 + cfg))
        K = N = 4096
        x = rng.standard_normal((M, K)).astype(np.float32)
        d = {"x": sha(x)}
        for i, R in enumerate(ranks):
            v = _pack_bits_le((1 - 2 * rng.integers(0, 2, size=(R, K))).astype(np.int8))
            u = _pack_bits_le((1 - 2 * rng.integers(0, 2, size=(N, R))).astype(np.int8))
            g = (np.abs(rng.standard_normal(K)) + 0.05).astype(np.float32)
            l = (np.abs(rng.standard_normal(R)) + 0.05).astype(np.float32)
            h = (np.abs(rng.standard_normal(N)) + 0.05).astype(np.float32)
            for key, a in (("v_sign", v), ("u_sign", u), ("g", g), ("l", l), ("h", h)):
                d[f"b{i}/{key}"] = sha(a)
        res[f"config{cfg}"] = {"M": M, "K": K, "N": N, "ranks": ranks, "sha256": d}
    return res


def main():
    (HERE / "pack_vectors.json").write_text(json.dumps(pack_vectors(), indent=1) + "\n")
    np.savez_compressed(HERE / "forward_small.npz", **forward_fixtures())
    (HERE / "synthetic_digests.json").write_text(json.dumps(synthetic_digests(), indent=1) + "\n")
    print("wrote", sorted(p.name for p in HERE.iterdir() if p.suffix in (".json", ".npz")))


if __name__ == "__main__":
    main()
