"""The constants of the forward kernels' table sin/cos (`sin_cos_tab` in
cufk_amd/csrc/chain_ops.h), read from the source and checked against numpy's sin/cos.

The kernels evaluate, for a float angle x in double:
    t = fma(x, 64/pi, 1.5 * 2^52),  k = t - 1.5 * 2^52,  r = fma(-k, pi/64, x),  u = r^2,
    sin r = r + s1 r u,  w = u (c2 u - 1/2),
    sin x = T_s[k] + T_s[k] w + T_c[k] sin r,  cos x = T_c[k] + T_c[k] w - T_s[k] sin r,
with (T_s, T_c)[j] = (sin, cos)(j pi/64) from a 128-entry table indexed by k mod 128.  This
test evaluates the same steps in float64 (without fused multiply-adds, which moves results by
an ulp, far below the bars) with the constants parsed from the source, so a mistyped constant
or table entry fails it.  Bars: |error| <= 1e-11 for sin and cos over |x| <= 2 pi (dihedrals
and bond angles; the cubic's equal-ripple bound is 9.72e-12) and <= 2e-11 up to |x| = 65536
(the kernels' polynomial range, where the one-part reduction adds up to |k| 2^-58), and
sin^2 + cos^2 within 2e-12 of 1 (a bias of that norm is what would shrink a long float chain).
The Taylor cubic (s1 = -1/6) misses the first bar, which is what the minimax coefficient buys.
"""

from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

SRC = Path(__file__).resolve().parent.parent / "cufk_amd" / "csrc" / "chain_ops.h"


def _constants():
    text = SRC.read_text()
    body = text[text.index("void sin_cos_tab(float xf"):]
    body = body[: body.index("\n}\n")]
    num = r"(-?\d+\.\d+(?:e-?\d+)?)"
    k_round = float(re.search(r"kRound = " + num, body).group(1))
    inv_step = float(re.search(r"fma\(x, " + num + r", kRound\)", body).group(1))
    step = float(re.search(r"fma\(-k, " + num + r", x\)", body).group(1))
    s1 = float(re.search(r"fma\(r \* u, " + num + r", r\)", body).group(1))
    c2 = float(re.search(r"fma_sk_minus_half\(u, " + num + r"\)", body).group(1))
    table_src = text[text.index("kTable[kSinCosTable][2] = {"):]
    table_src = table_src[: table_src.index("};")]
    table = np.array([[float(a), float(b)] for a, b in re.findall(r"\{" + num + r", " + num + r"\}", table_src)])
    return k_round, inv_step, step, s1, c2, table


def _sin_cos(x, k_round, inv_step, step, s1, c2, table):
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    t = x * inv_step + k_round
    k = t - k_round
    r = x - k * step
    u = r * r
    sr = r + (r * u) * s1
    w = u * (u * c2 - 0.5)
    idx = (t.view(np.uint64) & np.uint64(127)).astype(np.int64)
    ts, tc = table[idx, 0], table[idx, 1]
    return ts + ts * w + tc * sr, tc + tc * w - ts * sr


def _angles(wide=False):
    rng = np.random.default_rng(5)
    if wide:
        return rng.uniform(-65536.0, 65536.0, 200_000).astype(np.float32)  # the polynomial range
    return np.concatenate([
        rng.uniform(-np.pi, np.pi, 200_000),          # dihedrals
        rng.normal(2.05, 0.2, 100_000),               # bond angles
        np.linspace(-2 * np.pi, 2 * np.pi, 100_001),  # every table interval, both signs
    ]).astype(np.float32)


def test_table_has_the_exact_values():
    from mpmath import cos, mp, pi, sin

    *_, table = _constants()
    assert table.shape == (128, 2)
    mp.dps = 40
    for j in range(128):  # correctly rounded (sin, cos)(j pi / 64); the zeros exact
        assert abs(table[j, 0] - float(sin(j * pi / 64))) <= 1e-38, j
        assert abs(table[j, 1] - float(cos(j * pi / 64))) <= 1e-38, j


def test_reduction_constants():
    k_round, inv_step, step, *_ = _constants()
    assert k_round == 1.5 * 2.0**52
    assert inv_step == 64 / np.pi and step == np.pi / 64


@pytest.mark.parametrize("wide,bar", [(False, 1e-11), (True, 2e-11)])
def test_table_sin_cos_accuracy_and_norm(wide, bar):
    c = _constants()
    x = _angles(wide)
    s, co = _sin_cos(x, *c)
    xd = x.astype(np.float64)
    es, ec = np.abs(s - np.sin(xd)), np.abs(co - np.cos(xd))
    print(f"max |sin err| {es.max():.2e}, max |cos err| {ec.max():.2e}")
    assert es.max() <= bar and ec.max() <= bar
    assert np.abs(s * s + co * co - 1.0).max() <= 2e-12


def test_taylor_cubic_would_fail_the_bar():
    k_round, inv_step, step, _s1, c2, table = _constants()
    x = _angles()
    s, _ = _sin_cos(x, k_round, inv_step, step, -1.0 / 6.0, c2, table)
    assert np.abs(s - np.sin(x.astype(np.float64))).max() > 1e-11


@pytest.mark.parametrize("entry", [3, 77])
def test_a_wrong_table_entry_is_caught(entry):
    k_round, inv_step, step, s1, c2, table = _constants()
    bad = table.copy()
    bad[entry, 0] += 1e-9
    x = _angles()
    s, _ = _sin_cos(x, k_round, inv_step, step, s1, c2, bad)
    assert np.abs(s - np.sin(x.astype(np.float64))).max() > 1e-11
