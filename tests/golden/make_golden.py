"""Write the golden fixtures of the FP8 linear path (``fp8_golden.npz``).

The reference ships no test vectors for this path and cannot be imported here, so the
expected values are computed by code written independently of both the torch oracle
and the HIP kernels: plain numpy, with

* e4m3 encoding by nearest-value search over the 256-code table built from the OCP
  bit layout (ties to the even code), after the reference's clamp to +-448
  (reference quant.py:19-79);
* fp32 scales by numpy's IEEE fp32 division, as the reference computes them;
* MX exponents as ceil of the fp32-rounded log2 (reference quant.py:40-56);
* matrix products in float64 (reference gemm.py:17-189), with the W8A16 M > 1
  dequantized weight rounded to bf16 first (reference gemm.py:95-126).

Run ``python tests/golden/make_golden.py`` to regenerate; the output is deterministic.
"""

from __future__ import annotations

import pathlib

import numpy as np

OUT = pathlib.Path(__file__).resolve().parent / "fp8_golden.npz"
RNG = np.random.default_rng(20261201)


# ------------------------------------------------------------------ codecs
def e4m3_table() -> np.ndarray:
    """fp64 value of every e4m3fn code (NaN for 0x7F / 0xFF)."""
    v = np.empty(256)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 3) & 0xF, c & 7
        if e == 0xF and m == 7:
            v[c] = np.nan
        elif e == 0:
            v[c] = s * m * 2.0**-9
        else:
            v[c] = s * (1 + m / 8) * 2.0 ** (e - 7)
    return v


TABLE = e4m3_table()
POS = TABLE[:127]  # codes 0x00..0x7E, increasing


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """fp32/fp64 values -> e4m3 codes: clamp to +-448, nearest value, ties to even."""
    x = np.asarray(x, dtype=np.float64)
    mag = np.minimum(np.abs(x), 448.0)
    hi = np.clip(np.searchsorted(POS, mag), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    dlo, dhi = mag - POS[lo], POS[hi] - mag
    pick = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo % 2 == 0, lo, hi)))
    return (pick | np.where(np.signbit(x), 0x80, 0)).astype(np.uint8)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 values -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def e8m0_value(codes: np.ndarray) -> np.ndarray:
    return np.where(codes == 0xFF, np.nan, (codes.astype(np.uint32) << 23).view(np.float32).astype(np.float64))


# ------------------------------------------------------------------ inputs
_MIDS = (POS[:-1] + POS[1:]) / 2  # the 126 midpoints between positive e4m3 values


def quant_input() -> np.ndarray:
    """[8, 256] bf16 rows exercising the quantizers' corner cases."""
    rows = [
        np.zeros(256),                                              # amax floor 1e-10
        np.full(256, -3.0),                                         # single value: q = -448
        RNG.standard_normal(256),                                   # plain
        np.where(np.arange(256) == 77, 300.0, 1e-3 * RNG.standard_normal(256)),  # outlier: subnormals
        np.concatenate([[448.0], _MIDS, -_MIDS, np.zeros(3)]),     # exact ties at scale 1
        RNG.standard_t(3, 256) * 1e4,                               # heavy tail, large
        RNG.standard_normal(256) * 1e-30,                           # tiny (MX clamp region)
        np.concatenate([np.zeros(128), RNG.standard_normal(128)]),  # one zero group
    ]
    return bf16_bits(np.stack(rows).astype(np.float32))


def mx_boundary_input() -> np.ndarray:
    """[4, 128] fp32 rows whose 32-groups have amax at or just above 448 * 2^k."""
    rows = []
    for base in (-20, -3, 0, 9):
        row = []
        for j, steps in enumerate((0, 1, 2, 3)):
            amax = np.float32(448.0 * 2.0 ** (base + j))
            for _ in range(steps):
                amax = np.nextafter(amax, np.float32(np.inf))
            g = (RNG.standard_normal(32) * 0.1 * amax).astype(np.float32)
            g[j] = -amax
            row.append(g)
        rows.append(np.concatenate(row))
    return np.stack(rows).astype(np.float32)


# ------------------------------------------------------------------ expected quant
def per_token(x: np.ndarray, group: int) -> tuple[np.ndarray, np.ndarray]:
    m, k = x.shape
    g = x.reshape(m, k // group, group)
    s = (np.maximum(np.abs(g).max(-1), np.float32(1e-10)) / np.float32(448.0)).astype(np.float32)
    q = e4m3_encode((g / s[..., None]).astype(np.float32))
    return q.reshape(m, k), s


def mx(x: np.ndarray, group: int = 32) -> tuple[np.ndarray, np.ndarray]:
    m, k = x.shape
    g = x.reshape(m, k // group, group)
    amax = np.abs(g).max(-1).astype(np.float32)
    r = np.maximum(amax / np.float32(448.0), np.float32(1e-38)).astype(np.float32)
    e = np.clip(np.ceil(np.log2(r.astype(np.float64)).astype(np.float32)), -126, 127)
    zero = amax == 0
    code = np.where(zero, 0, e + 127).astype(np.uint8)
    scale = np.where(zero, 1.0, 2.0 ** e.astype(np.float64))
    q = np.where(zero[..., None], 0, e4m3_encode((g.astype(np.float64) / scale[..., None]).astype(np.float32)))
    return q.astype(np.uint8).reshape(m, k), code


# ------------------------------------------------------------------ expected products
def rand_codes(shape) -> np.ndarray:
    """Random finite e4m3 codes (no NaN)."""
    c = RNG.integers(0, 256, size=shape, dtype=np.uint8)
    return np.where((c & 0x7F) == 0x7F, c ^ 1, c).astype(np.uint8)


def main() -> None:
    fx: dict[str, np.ndarray] = {}
    xq = quant_input()
    xf = bf16_value(xq)
    fx["quant_x_bf16"] = xq
    fx["pt_q"], s = per_token(xf, 256)
    fx["pt_s"] = s[:, 0]
    fx["g128_q"], fx["g128_s"] = per_token(xf, 128)
    fx["mx_q"], fx["mx_code"] = mx(xf)
    xb = mx_boundary_input()
    fx["mxb_x_f32"] = xb
    fx["mxb_q"], fx["mxb_code"] = mx(xb)

    # fp8_scaled_mm (rowwise): out = (a @ b^T) * sa * sb + bias
    a, b = rand_codes((5, 64)), rand_codes((24, 64))
    sa, sb = RNG.uniform(1e-3, 1e-2, 5).astype(np.float32), RNG.uniform(1e-3, 1e-2, 24).astype(np.float32)
    bias = bf16_value(bf16_bits(RNG.standard_normal(24).astype(np.float32)))
    fx.update(smm_a=a, smm_b=b, smm_sa=sa, smm_sb=sb, smm_bias=bias)
    fx["smm_out"] = (TABLE[a] @ TABLE[b].T) * sa[:, None].astype(np.float64) * sb[None, :] + bias[None, :]

    # fp8_blockwise_mm: per-128 K blocks, [M, K/128] and [ceil(N/128), K/128] scales
    a, b = rand_codes((3, 256)), rand_codes((130, 256))
    sa = RNG.uniform(1e-3, 1e-1, (3, 2)).astype(np.float32)
    sb = RNG.uniform(1e-3, 1e-1, (2, 2)).astype(np.float32)
    fx.update(bmm_a=a, bmm_b=b, bmm_sa=sa, bmm_sb=sb)
    out = np.zeros((3, 130))
    for kb in range(2):
        part = TABLE[a[:, kb * 128:(kb + 1) * 128]] @ TABLE[b[:, kb * 128:(kb + 1) * 128]].T
        out += part * sa[:, kb:kb + 1] * np.repeat(sb[:, kb], 128)[None, :130]
    fx["bmm_out"] = out

    # mxfp8_scaled_mm: per-32 UE8M0 codes on both operands, bias added
    a, w = rand_codes((3, 64)), rand_codes((20, 64))
    ca, cw = RNG.integers(120, 135, (3, 2), dtype=np.uint8), RNG.integers(120, 135, (20, 2), dtype=np.uint8)
    bias = RNG.standard_normal(20).astype(np.float32)
    fx.update(mxm_a=a, mxm_w=w, mxm_ca=ca, mxm_cw=cw, mxm_bias=bias)
    ad = TABLE[a] * np.repeat(e8m0_value(ca), 32, axis=1)
    wd = TABLE[w] * np.repeat(e8m0_value(cw), 32, axis=1)
    fx["mxm_out"] = ad @ wd.T + bias[None, :]

    # W8A16: per-row fp32, block-128 fp32, and per-32 UE8M0 weight scales
    k, n = 256, 40
    w = rand_codes((n, k))
    xg = bf16_bits((RNG.standard_normal((3, k))).astype(np.float32))
    fx.update(w16_w=w, w16_x_bf16=xg)
    scales = {
        "row": (RNG.uniform(1e-3, 1e-2, (n, 1)).astype(np.float32), 1, k),
        "b128": (RNG.uniform(1e-3, 1e-2, (1, 2)).astype(np.float32), 128, 128),
        "e8m0": (RNG.integers(115, 125, (n, k // 32), dtype=np.uint8), 1, 32),
    }
    for name, (sc, by, bx) in scales.items():
        fx[f"w16_{name}_scale"] = sc
        sv = e8m0_value(sc) if sc.dtype == np.uint8 else sc.astype(np.float64)
        smat = sv[np.arange(n)[:, None] // by, np.arange(k)[None, :] // bx]
        deq = TABLE[w] * smat
        xv = bf16_value(xg).astype(np.float64)
        fx[f"w16_{name}_gemv"] = deq @ xv[0]                                   # M == 1 (gemm.py:129-157)
        deq16 = bf16_value(bf16_bits(deq.astype(np.float32))).astype(np.float64)
        fx[f"w16_{name}_gemm"] = xv @ deq16.T                                  # M > 1 (gemm.py:95-126)
    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(fx)} arrays)")


if __name__ == "__main__":
    main()
