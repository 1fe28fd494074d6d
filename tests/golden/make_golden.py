"""Generate the golden fixtures in this directory.

    python tests/golden/make_golden.py

Every expected output here is computed by this file alone, in float64 numpy,
from the textbook definitions; nothing is taken from the oracle, the HIP
library or torch. The tests then hold both the oracle and the HIP kernels to
these numbers:

  e4m3_table.npz         all 256 OCP E4M3 codes decoded from the format's
                         definition (bias 7, S.1111.111 = NaN, no inf)
  attn_c1_fp32.npz       config 1: fp32, non-causal MHA, B1 H1 S128 D64
  attn_f16_mha.npz       the reference tile program's dtype (f16), non-causal
  attn_bf16_causal_gqa.npz  bf16, causal, 4 query heads on 2 KV heads,
                         ragged S = 40
  decode_bf16_gqa.npz    split-K decode, bf16 KV, 8 query heads on 2 KV heads
  decode_fp8.npz         the same query on E4M3 KV with per-32-token scales
                         (codes and scales quantised here), expected output
                         from the dequantised values
  scan_small.npz         Mamba-1 selective scan with z, D and delta_bias
  scan_plain.npz         the scan without z, D, bias and without softplus

Expected outputs with two or more dimensions are stored as float32.
Inputs are N(0, 1) from numpy's PCG64 with fixed seeds, rounded once to the
storage dtype (bf16 by round-to-nearest-even on the fp32 bits, f16 by
numpy's cast); the closed forms run on the rounded values. The reference
(Evan-Zhao/mlir-toy) ships no numeric vectors (its goldens are emitted
source text), so these are the build's own.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


# ------------------------------------------------------------------ codecs


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float -> bf16 storage bits, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def e4m3_table() -> np.ndarray:
    """Value of every E4M3 code: sign, 4 exponent bits (bias 7), 3 mantissa
    bits; exponent 0 is subnormal (m/8 * 2^-6); S.1111.111 is NaN."""
    vals = np.empty(256, dtype=np.float64)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            vals[c] = np.nan
        elif e == 0:
            vals[c] = s * (m / 8.0) * 2.0 ** -6
        else:
            vals[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """Nearest E4M3 code by exhaustive search over the positive codes, ties to
    the even code, saturating at +-448 (the OCP 'saturate' conversion)."""
    table = e4m3_table()
    pos = table[:0x7F]                        # codes 0x00..0x7e, ascending
    x = np.asarray(x, dtype=np.float64)
    a = np.minimum(np.abs(x), 448.0)
    d = np.abs(a[..., None] - pos)            # distance to every code
    best = d.min(axis=-1, keepdims=True)
    cand = d == best
    # among equally near codes take the one with an even mantissa
    even = (np.arange(0x7F) & 1) == 0
    pick = np.where((cand & even).any(axis=-1), np.argmax(cand & even, axis=-1),
                    np.argmax(cand, axis=-1))
    code = pick.astype(np.uint8)
    # the sign bit is kept also when the magnitude rounds to zero (-0 = 0x80)
    return np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)


# ----------------------------------------------------------- closed forms


def attention(q, k, v, causal: bool, scale: float):
    """softmax(q k^T scale) v per (b, h) in float64; KV head = h // group;
    causal keeps key j <= query i (S_q == S_kv). Returns (o, lse natural)."""
    B, Hq, Sq, D = q.shape
    Hk = k.shape[1]
    g = Hq // Hk
    o = np.empty((B, Hq, Sq, D))
    lse = np.empty((B, Hq, Sq))
    for b in range(B):
        for h in range(Hq):
            s = q[b, h] @ k[b, h // g].T * scale
            if causal:
                s = np.where(np.tril(np.ones((Sq, k.shape[2]), dtype=bool)), s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            p = np.exp(s - m)
            l = p.sum(axis=1, keepdims=True)
            o[b, h] = (p / l) @ v[b, h // g]
            lse[b, h] = (m + np.log(l))[:, 0]
    return o, lse


def decode(q, k, v, scale: float):
    """One query row per head against all L keys (float64)."""
    B, Hq, D = q.shape
    o, lse = attention(q[:, :, None, :], k, v, False, scale)
    return o[:, :, 0, :], lse[:, :, 0]


def selective_scan(u, dr, A, Bm, Cm, D, z, bias, softplus: bool):
    """Sequential Mamba-1 recurrence in float64 (Gu & Dao 2023, zero-order
    hold with B_bar = delta B): x <- exp(delta A) x + delta B u,
    y = (C.x + D u) * silu(z)."""
    b_, dm, L = u.shape
    n = A.shape[1]
    y = np.empty((b_, dm, L))
    for b in range(b_):
        for c in range(dm):
            x = np.zeros(n)
            for t in range(L):
                v = dr[b, c, t] + (bias[c] if bias is not None else 0.0)
                dl = (v if v > 20.0 else np.log1p(np.exp(v))) if softplus else v
                x = np.exp(dl * A[c]) * x + dl * Bm[b, :, t] * u[b, c, t]
                acc = float(Cm[b, :, t] @ x)
                if D is not None:
                    acc += D[c] * u[b, c, t]
                if z is not None:
                    zz = z[b, c, t]
                    acc *= zz / (1.0 + np.exp(-zz))
                y[b, c, t] = acc
    return y


# ---------------------------------------------------------------- fixtures


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def make_all() -> dict[str, dict[str, np.ndarray]]:
    out: dict[str, dict[str, np.ndarray]] = {}

    codes = np.arange(256, dtype=np.uint8)
    out["e4m3_table"] = {"codes": codes, "values": e4m3_table()}

    # config 1: fp32 MHA B1 H1 S128 D64, non-causal, scale 1/sqrt(D)
    r = _rng(1)
    q, k, v = (r.standard_normal((1, 1, 128, 64)).astype(np.float32) for _ in range(3))
    o, lse = attention(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                       False, 1.0 / np.sqrt(64))
    out["attn_c1_fp32"] = {"q": q, "k": k, "v": v, "o": o, "lse": lse,
                           "causal": np.array(0), "scale": np.array(1.0 / np.sqrt(64))}

    # the reference program's dtype: f16, non-causal MHA, D = 64
    r = _rng(2)
    q, k, v = (r.standard_normal((1, 2, 64, 64)).astype(np.float16) for _ in range(3))
    o, lse = attention(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                       False, 1.0 / np.sqrt(64))
    out["attn_f16_mha"] = {"q": q, "k": k, "v": v, "o": o, "lse": lse,
                           "causal": np.array(0), "scale": np.array(1.0 / np.sqrt(64))}

    # bf16, causal, GQA 4:2, ragged S = 40, D = 128
    r = _rng(3)
    qb = bf16_bits(r.standard_normal((1, 4, 40, 128)))
    kb = bf16_bits(r.standard_normal((1, 2, 40, 128)))
    vb = bf16_bits(r.standard_normal((1, 2, 40, 128)))
    o, lse = attention(bf16_value(qb), bf16_value(kb), bf16_value(vb), True,
                       1.0 / np.sqrt(128))
    out["attn_bf16_causal_gqa"] = {"q": qb, "k": kb, "v": vb, "o": o, "lse": lse,
                                   "causal": np.array(1),
                                   "scale": np.array(1.0 / np.sqrt(128))}

    # split-K decode: B2, 8 query heads on 2 KV heads, L = 96, D = 128
    r = _rng(4)
    qb = bf16_bits(r.standard_normal((2, 8, 128)))
    kb = bf16_bits(r.standard_normal((2, 2, 96, 128)))
    vb = bf16_bits(r.standard_normal((2, 2, 96, 128)))
    o, lse = decode(bf16_value(qb), bf16_value(kb), bf16_value(vb), 1.0 / np.sqrt(128))
    out["decode_bf16_gqa"] = {"q": qb, "k": kb, "v": vb, "o": o, "lse": lse,
                              "num_splits": np.array(3), "scale": np.array(1.0 / np.sqrt(128))}

    # fp8 KV of the same K/V: per (b, kv head, 32-token block) scale
    # amax / 448, codes = E4M3(x * (448 / amax)) in fp32 arithmetic
    sb = 32
    kv = {"k": kb, "v": vb}
    fp8: dict[str, np.ndarray] = {"q": qb, "scale_block": np.array(sb)}
    deq = {}
    for name, bits in kv.items():
        x = (bits.astype(np.uint32) << 16).view(np.float32)
        B, Hk, L, D = x.shape
        nsb = -(-L // sb)
        cds = np.empty(x.shape, dtype=np.uint8)
        scl = np.empty((B, Hk, nsb), dtype=np.float32)
        for blk in range(nsb):
            xs = x[:, :, blk * sb:(blk + 1) * sb, :]
            amax = np.abs(xs).max(axis=(2, 3)).astype(np.float32)
            inv = np.float32(448.0) / amax
            scl[:, :, blk] = amax / np.float32(448.0)
            cds[:, :, blk * sb:(blk + 1) * sb, :] = e4m3_encode(
                (xs * inv[:, :, None, None]).astype(np.float32))
        fp8[name + "_codes"] = cds
        fp8[name + "_scale"] = scl
        deq[name] = e4m3_table()[cds] * np.repeat(scl.astype(np.float64), sb, axis=2)[:, :, :L, None]
    o8, lse8 = decode(bf16_value(qb), deq["k"], deq["v"], 1.0 / np.sqrt(128))
    fp8.update({"o": o8, "lse": lse8, "o_bf16_kv": o, "num_splits": np.array(3),
                "scale": np.array(1.0 / np.sqrt(128))})
    out["decode_fp8"] = fp8

    # selective scan with z, D and bias (softplus on); ragged L = 40
    r = _rng(5)
    bsz, dm, L, n = 2, 8, 40, 16
    u, dr, z = (bf16_bits(r.standard_normal((bsz, dm, L))) for _ in range(3))
    Bm, Cm = (bf16_bits(r.standard_normal((bsz, n, L))) for _ in range(2))
    A = (-np.exp(r.standard_normal((dm, n)))).astype(np.float32)
    D = r.standard_normal(dm).astype(np.float32)
    bias = r.standard_normal(dm).astype(np.float32)
    y = selective_scan(bf16_value(u), bf16_value(dr), A.astype(np.float64), bf16_value(Bm),
                       bf16_value(Cm), D.astype(np.float64), bf16_value(z),
                       bias.astype(np.float64), True)
    out["scan_small"] = {"u": u, "delta": dr, "A": A, "B": Bm, "C": Cm, "D": D, "z": z,
                         "delta_bias": bias, "y": y}

    # plain scan: no z, no D, no bias, delta used as given (made positive)
    r = _rng(6)
    bsz, dm, L = 1, 4, 24
    u = bf16_bits(r.standard_normal((bsz, dm, L)))
    dr = bf16_bits(np.abs(r.standard_normal((bsz, dm, L))) * 0.5)
    Bm, Cm = (bf16_bits(r.standard_normal((bsz, n, L))) for _ in range(2))
    A = (-np.exp(r.standard_normal((dm, n)))).astype(np.float32)
    y = selective_scan(bf16_value(u), bf16_value(dr), A.astype(np.float64), bf16_value(Bm),
                       bf16_value(Cm), None, None, None, False)
    out["scan_plain"] = {"u": u, "delta": dr, "A": A, "B": Bm, "C": Cm, "y": y}
    return out


def main() -> None:
    for name, arrays in make_all().items():
        # expected outputs are kept in float32 (|relative error| <= 6e-8, far
        # inside every tolerance the tests apply) to keep the files small
        arrays = {k: (a.astype(np.float32) if a.dtype == np.float64 and a.ndim > 1 else a)
                  for k, a in arrays.items()}
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        size = (HERE / f"{name}.npz").stat().st_size
        print(f"{name}.npz  {size / 1024:.1f} KiB")


if __name__ == "__main__":
    main()
