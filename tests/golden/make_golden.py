"""Generate the committed golden fixtures for MatMulNBits (run from the repo root).

    python tests/golden/make_golden.py

The reference holds no stored output vectors for this path (its ledger records MATCH verdicts
only, ``evidence/proof_ledger.jsonl:128-133``), so the fixtures here are built from first
principles, independently of the numpy oracle:

* ``kat_*`` — integer-exact known answers in the construction of the reference's interpreter
  test (``bench/test_weight_reread.py:71-108``): A in {-4..4}, weights uniform over the bit
  range, scales in {1/8, 2/8, 3/8}.  Every partial sum is a multiple of 1/8 far below 2^24, so
  the answer is independent of summation order and the expected values are computed here with
  exact rational arithmetic (``fractions.Fraction``), element by element, from the packed
  bytes — no numpy dequant, no oracle code.  Magnitudes stay below 2^20, so any fp32
  accumulation is exact and the fp16 output is the single round-half-even of the exact value
  (the reference asserts ``max diff == 0`` for this construction, ``:114-126``).
* ``dequant_*`` — the fp16 dequant of random packed inputs, computed per element as
  ``struct.pack('e', float(Fraction))`` (IEEE binary16, round-half-even) of the exact rational
  ``(q - zp) * s``, with the IEEE sign of a zero product (a negative ``q - zp`` times a zero
  scale is ``-0``).

Each fixture stores its inputs and expected outputs as arrays (data only).
"""

from __future__ import annotations

import struct
import sys
from fractions import Fraction
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent


def _pack(q: np.ndarray, bits: int, bs: int) -> np.ndarray:
    """[N, K] values -> [N, K/bs, bs*bits/8] bytes, low nibble first (written independently)."""
    N, K = q.shape
    out = bytearray()
    for n in range(N):
        for blk in range(K // bs):
            vals = [int(v) for v in q[n, blk * bs:(blk + 1) * bs]]
            if bits == 4:
                for i in range(0, bs, 2):
                    out.append(vals[i] | (vals[i + 1] << 4))
            else:
                out.extend(vals)
    return np.frombuffer(bytes(out), dtype=np.uint8).reshape(N, K // bs, bs * bits // 8).copy()


def _pack_zp(z: np.ndarray, bits: int) -> np.ndarray:
    N, bpc = z.shape
    per = (bpc * bits + 7) // 8
    out = np.zeros((N, per), dtype=np.uint8)
    for n in range(N):
        for blk in range(bpc):
            v = int(z[n, blk])
            if bits == 4:
                out[n, blk // 2] |= (v << 4) if (blk & 1) else v
            else:
                out[n, blk] = v
    return out


def _byte_q(Bp: np.ndarray, n: int, k: int, bits: int, bs: int) -> int:
    blob = bs * bits // 8
    flat = Bp.reshape(Bp.shape[0], -1)
    blk, i = divmod(k, bs)
    if bits == 4:
        byte = int(flat[n, blk * blob + i // 2])
        return (byte >> 4) if (i & 1) else (byte & 0xF)
    return int(flat[n, blk * blob + i])


def _byte_zp(zp, n: int, blk: int, bits: int) -> int:
    if zp is None:
        return 1 << (bits - 1)
    if bits == 4:
        byte = int(zp[n, blk // 2])
        return (byte >> 4) if (blk & 1) else (byte & 0xF)
    return int(zp[n, blk])


def _half_bits(x: Fraction, negative_zero: bool = False) -> int:
    v = float(x)
    if v == 0.0 and negative_zero:
        v = -0.0
    return struct.unpack("<H", struct.pack("<e", v))[0]


def kat(name: str, M: int, N: int, K: int, bits: int, bs: int, with_zp: bool, seed: int):
    rng = np.random.default_rng(seed)
    bpc = K // bs
    A = rng.integers(-4, 5, size=(M, K))
    q = rng.integers(0, 1 << bits, size=(N, K))
    s8 = rng.integers(1, 4, size=(N, bpc))                         # scale = s8 / 8
    Bp = _pack(q.astype(np.uint8), bits, bs)
    zp = _pack_zp(rng.integers(0, 1 << bits, size=(N, bpc)), bits) if with_zp else None
    Y = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            acc = Fraction(0)
            for k in range(K):
                blk = k // bs
                w = (_byte_q(Bp, n, k, bits, bs) - _byte_zp(zp, n, blk, bits)) * Fraction(int(s8[n, blk]), 8)
                acc += int(A[m, k]) * w
            assert abs(acc) < (1 << 20) and (acc * 8).denominator == 1
            Y[m, n] = float(acc)
    arrays = dict(A=A.astype(np.float16), B=Bp, scales=(s8.reshape(-1) / 8.0).astype(np.float16),
                  Y=Y.astype(np.float16), Y_exact=Y,
                  meta=np.array([M, N, K, bits, bs, int(with_zp)], dtype=np.int64))
    if zp is not None:
        arrays["zp"] = zp
    np.savez_compressed(OUT / f"{name}.npz", **arrays)


def dequant(name: str, N: int, K: int, bits: int, bs: int, with_zp: bool, seed: int):
    rng = np.random.default_rng(seed)
    bpc = K // bs
    q = rng.integers(0, 1 << bits, size=(N, K)).astype(np.uint8)
    Bp = _pack(q, bits, bs)
    # scales spread over fp16 magnitudes, including values whose products round
    s = (np.abs(rng.standard_normal(N * bpc)) * 0.02).astype(np.float16)
    s[:4] = np.array([0.02, 1.0 / 3.0, 6.1e-5, 0.0], dtype=np.float16)
    zp = _pack_zp(rng.integers(0, 1 << bits, size=(N, bpc)), bits) if with_zp else None
    W = np.zeros((N, K), dtype=np.uint16)
    for n in range(N):
        for k in range(K):
            blk = k // bs
            d = _byte_q(Bp, n, k, bits, bs) - _byte_zp(zp, n, blk, bits)
            sv = float(s[n * bpc + blk])
            # IEEE: a zero product carries the XOR of the operands' signs ((float)0 is +0)
            W[n, k] = _half_bits(d * Fraction(sv), negative_zero=(d < 0) != (np.signbit(sv)))
    arrays = dict(B=Bp, scales=s, W_bits=W, meta=np.array([N, K, bits, bs, int(with_zp)], dtype=np.int64))
    if zp is not None:
        arrays["zp"] = zp
    np.savez_compressed(OUT / f"{name}.npz", **arrays)


def main() -> int:
    # the reference's own interpreter case: K=64, N=8, bs=32, 4-bit (bench/test_weight_reread.py:120)
    kat("kat_k64_n8_b4_bs32", 1, 8, 64, 4, 32, False, 7)
    kat("kat_k64_n130_b4_bs32_m3", 3, 130, 64, 4, 32, False, 8)
    kat("kat_k128_n48_b4_bs16_zp", 2, 48, 128, 4, 16, True, 9)
    kat("kat_k256_n40_b4_bs64_zp_m5", 5, 40, 256, 4, 64, True, 10)
    kat("kat_k256_n33_b4_bs128", 4, 33, 256, 4, 128, False, 11)
    kat("kat_k64_n24_b8_bs32_zp", 2, 24, 64, 8, 32, True, 12)
    kat("kat_k64_n17_b8_bs16", 3, 17, 64, 8, 16, False, 13)
    kat("kat_k384_n64_b4_bs32_zp_m17", 17, 64, 384, 4, 32, True, 14)
    for bits in (4, 8):
        for bs in (16, 32, 64, 128):
            for zp in (False, True):
                dequant(f"dequant_b{bits}_bs{bs}{'_zp' if zp else ''}", 6, 256, bits, bs, zp,
                        100 + bits * 10 + bs + int(zp))
    print("wrote fixtures to", OUT)
    return 0


if __name__ == "__main__":
    sys.exit(main())
