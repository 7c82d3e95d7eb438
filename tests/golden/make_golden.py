"""Writes the committed fixtures under tests/golden/.

1. kat_q4k.npz / kat_q5k.npz / kat_q6k.npz -- known-answer blocks.  Each
   block is PACKED from intended field values (scales, mins, quants, d) by
   the GGUF super-block packing rules written element-major below, and its
   expected dequantized values are computed from those intended values in
   float64 -- without the oracle's unpack code.  A transposed nibble, a
   wrong qh bit, a wrong Q6_K scale index or a lost high scale bit makes the
   oracle (and the GPU) disagree with these blocks.
2. seeded_small.npz -- small seeded workloads and the oracle's outputs on
   them: a regression record of the oracle itself, used by the GPU parity
   tests at sizes that need no CPU time.

Run from the repo root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "recursive-routing-racer-rs_amd"))

F16 = {1.0: 0x3C00, 0.5: 0x3800, 0.25: 0x3400, 0.0: 0x0000, 2.0: 0x4000}


# ---- packing rules (element-major statements of the GGUF K-quant layouts) ----

def pack_scales_k4(sc, mn):
    """8 six-bit scales and mins -> the 12 packed bytes of Q4_K/Q5_K."""
    q = np.zeros(12, np.uint8)
    for j in range(4):
        q[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return q


def pack_q4k(d16, dmin16, sc, mn, q):
    """q: 256 values 0..15; element e = 32*sub + j lives in qs[32*(sub//2) + j],
    low nibble for even sub, high nibble for odd sub."""
    b = np.zeros(144, np.uint8)
    b[0:2] = [d16 & 255, d16 >> 8]
    b[2:4] = [dmin16 & 255, dmin16 >> 8]
    b[4:16] = pack_scales_k4(sc, mn)
    for e in range(256):
        sub, j = divmod(e, 32)
        i = 16 + 32 * (sub // 2) + j
        b[i] |= (q[e] & 15) << (4 * (sub & 1))
    return b


def pack_q5k(d16, dmin16, sc, mn, q):
    """q: 256 values 0..31; low 4 bits as Q4_K, bit 4 of element 32*sub + j is
    bit `sub` of qh[j]."""
    b = np.zeros(176, np.uint8)
    b[0:2] = [d16 & 255, d16 >> 8]
    b[2:4] = [dmin16 & 255, dmin16 >> 8]
    b[4:16] = pack_scales_k4(sc, mn)
    for e in range(256):
        sub, j = divmod(e, 32)
        b[48 + 32 * (sub // 2) + j] |= (q[e] & 15) << (4 * (sub & 1))
        b[16 + j] |= ((q[e] >> 4) & 1) << sub
    return b


def pack_q6k(d16, sc, q):
    """q: 256 stored values 0..63 (dequantized value q - 32); element
    e = 128 g + 32 u + l: low 4 bits in ql[64 g + l + 32 (u & 1)] (low nibble
    for u < 2, high for u >= 2), high 2 bits at bits 2u..2u+1 of qh[32 g + l];
    scale sc[e // 16] (int8)."""
    b = np.zeros(210, np.uint8)
    for e in range(256):
        g, r = divmod(e, 128)
        u, l = divmod(r, 32)
        b[64 * g + l + 32 * (u & 1)] |= (q[e] & 15) << (4 * (u >> 1))
        b[128 + 32 * g + l] |= ((q[e] >> 4) & 3) << (2 * u)
    b[192:208] = np.asarray(sc, np.int64).astype(np.int8).view(np.uint8)
    b[208:210] = [d16 & 255, d16 >> 8]
    return b


def f16val(bits):
    return float(np.array([bits], np.uint16).view(np.float16)[0])


def expect_k4(d16, dmin16, sc, mn, q):
    d, dmin = f16val(d16), f16val(dmin16)
    with np.errstate(invalid="ignore"):
        return np.array([q[e] * (d * sc[e // 32]) - dmin * mn[e // 32] for e in range(256)], np.float64)


def expect_q6k(d16, sc, q):
    d = f16val(d16)
    with np.errstate(invalid="ignore"):
        return np.array([(d * sc[e // 16]) * (int(q[e]) - 32) for e in range(256)], np.float64)


def make_kats():
    rng = np.random.default_rng(20261201)
    out = {}

    # ---- Q4_K ----
    blocks, exp = [], []
    ones, zeros = [1] * 8, [0] * 8
    q = np.array([(7 * e + 3) % 16 for e in range(256)])
    blocks.append(pack_q4k(F16[1.0], F16[0.0], ones, zeros, q)); exp.append(expect_k4(F16[1.0], F16[0.0], ones, zeros, q))
    q = np.arange(256) % 16
    blocks.append(pack_q4k(F16[1.0], F16[0.0], ones, zeros, q)); exp.append(expect_k4(F16[1.0], F16[0.0], ones, zeros, q))
    sc = [1, 5, 17, 33, 63, 40, 9, 50]
    mn = [2, 60, 31, 7, 48, 3, 62, 20]
    for d16, dm16 in ((F16[1.0], F16[1.0]), (F16[0.5], F16[0.25]), (F16[0.0], F16[1.0]), (F16[2.0], F16[0.5])):
        q = rng.integers(0, 16, 256)
        blocks.append(pack_q4k(d16, dm16, sc, mn, q)); exp.append(expect_k4(d16, dm16, sc, mn, q))
    # every 6-bit scale/min value at every position, high bits included
    for rep in range(8):
        sc = rng.integers(0, 64, 8); mn = rng.integers(0, 64, 8); q = rng.integers(0, 16, 256)
        blocks.append(pack_q4k(F16[1.0], F16[1.0], sc, mn, q)); exp.append(expect_k4(F16[1.0], F16[1.0], sc, mn, q))
    # f16 edge values of d: smallest subnormal, largest subnormal, +inf (0 * inf -> NaN)
    for d16 in (0x0001, 0x03FF, 0x7C00):
        q = np.arange(256) % 16
        blocks.append(pack_q4k(d16, F16[0.0], ones, zeros, q)); exp.append(expect_k4(d16, F16[0.0], ones, zeros, q))
    out["q4k"] = (np.stack(blocks), np.stack(exp).astype(np.float32))

    # ---- Q5_K ----
    blocks, exp = [], []
    for s in range(8):
        for j in range(32):
            q = np.zeros(256, np.int64)
            q[32 * s + j] = 16
            blocks.append(pack_q5k(F16[1.0], F16[0.0], ones, zeros, q)); exp.append(expect_k4(F16[1.0], F16[0.0], ones, zeros, q))
    for rep in range(8):
        sc = rng.integers(0, 64, 8); mn = rng.integers(0, 64, 8); q = rng.integers(0, 32, 256)
        blocks.append(pack_q5k(F16[1.0], F16[1.0], sc, mn, q)); exp.append(expect_k4(F16[1.0], F16[1.0], sc, mn, q))
    out["q5k"] = (np.stack(blocks), np.stack(exp).astype(np.float32))

    # ---- Q6_K ----
    blocks, exp = [], []
    sc = list(range(1, 17))
    q = np.zeros(256, np.int64)
    blocks.append(pack_q6k(F16[1.0], sc, q)); exp.append(expect_q6k(F16[1.0], sc, q))
    sc = [-128, 127, -1, 1, -64, 63, -32, 31, 2, -3, 5, -7, 11, -13, 17, -19]
    q = np.arange(256) % 64
    blocks.append(pack_q6k(F16[0.5], sc, q)); exp.append(expect_q6k(F16[0.5], sc, q))
    # one high-bit at a time: every (qh byte, bit) pair
    for byte in range(64):
        for bit in range(8):
            g, l = divmod(byte, 32)
            u = bit // 2
            q = np.zeros(256, np.int64)
            q[128 * g + 32 * u + l] = 16 << (bit & 1)
            blocks.append(pack_q6k(F16[1.0], [1] * 16, q)); exp.append(expect_q6k(F16[1.0], [1] * 16, q))
    for rep in range(8):
        sc = rng.integers(-128, 128, 16); q = rng.integers(0, 64, 256)
        blocks.append(pack_q6k(F16[0.25], sc, q)); exp.append(expect_q6k(F16[0.25], sc, q))
    out["q6k"] = (np.stack(blocks), np.stack(exp).astype(np.float32))
    return out


def make_seeded():
    import oracle.oracle as orc
    import rrr_hip.synth as syn
    seed = 7
    rec = {}
    shapes = {12: (512, 8), 13: (768, 6), 14: (1024, 4)}
    for qt, (K, N) in shapes.items():
        W = syn.weight(seed, 100 + qt, qt, K, N)
        X = syn.normal_f32(seed, 200 + qt, 4 * K)
        rec[f"w{qt}"] = W
        rec[f"x{qt}"] = X
        rec[f"deq{qt}"] = orc.dequant(qt, W, K * N)
        rec[f"y{qt}"] = orc.gemv(qt, W, X, K, N, 4)
        rec[f"y{qt}_f64"] = orc.gemv(qt, W, X, K, N, 4, f64=True)
    x = syn.normal_f32(seed, 300, 3072)
    g = syn.normal_f32(seed, 301, 3072, 1.0, 0.1)
    rec["norm_x"], rec["norm_g"], rec["norm_y"] = x, g, orc.rms_norm(x, g)
    gu = syn.normal_f32(seed, 302, 2 * 512)
    rec["silu_gu"], rec["silu_mid"] = gu, orc.silu_gate(gu, 512)
    K, V = 256, 120
    E = syn.normal_f32(seed, 303, V * K, 0.0, 0.02)
    xl = syn.normal_f32(seed, 304, K)
    rec["lg_E"], rec["lg_x"] = E, xl
    rec["lg_y"] = orc.logits(xl, E, K, V)
    return rec


def main():
    for name, (blocks, exp) in make_kats().items():
        np.savez_compressed(os.path.join(HERE, f"kat_{name}.npz"), blocks=blocks, expected=exp)
        print(f"kat_{name}.npz: {blocks.shape[0]} blocks")
    np.savez_compressed(os.path.join(HERE, "seeded_small.npz"), **make_seeded())
    print("seeded_small.npz written")


if __name__ == "__main__":
    main()
