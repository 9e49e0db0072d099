"""Constants of the acceptance kernels' f64 exp (seeker_amd/csrc/sh_exp.h),
checked against 60-digit decimal arithmetic: the 64 table entries are the
correctly rounded 2^(j/64), the Cody-Waite pair sums to ln2/64 far beyond f64
precision, and the reduction factor is 64/ln2."""
import re
from decimal import Decimal, getcontext
from pathlib import Path

HDR = Path(__file__).resolve().parents[1] / "seeker_amd" / "csrc" / "sh_exp.h"


def _text():
    return HDR.read_text()


def test_table_is_correctly_rounded_exp2():
    getcontext().prec = 60
    body = _text().split("#define SH_EXP2_TABLE_64", 1)[1].split("}", 1)[0]
    vals = [float.fromhex(h) for h in re.findall(r"0x[0-9a-f.]+p[+-]\d+", body)]
    assert len(vals) == 64
    for j, v in enumerate(vals):
        exact = Decimal(2) ** (Decimal(j) / 64)
        assert v == float(exact), j
        # correctly rounded: no other double is closer
        lo, hi = Decimal(v) - exact, exact - Decimal(v)
        ulp = Decimal(float.fromhex("0x1p-52"))
        assert abs(lo) <= ulp / 2 and abs(hi) <= ulp / 2, j


def test_reduction_constants():
    getcontext().prec = 60
    t = _text()
    get = lambda name: float.fromhex(re.search(name + r" = (0x[0-9a-f.]+p[+-]\d+);", t).group(1))
    ln2 = Decimal(2).ln()
    hi, lo, c = get("kLn2o64Hi"), get("kLn2o64Lo"), get("kExp64OverLn2")
    assert abs(Decimal(hi) + Decimal(lo) - ln2 / 64) < Decimal(10) ** -33
    assert c == float(64 / ln2)
    # the high part is ln2/64 rounded to f64 (the fused y - n*hi then needs <= 53 bits)
    assert hi == float(ln2 / 64)
