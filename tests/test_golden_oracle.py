"""The C oracle reproduces every committed golden fixture (made by the big-integer brute force)."""
import os

import numpy as np

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


def cases():
    z = np.load(GOLDEN, allow_pickle=False)
    for i in range(int(z["count"])):
        p = f"c{i:03d}_"
        t, rows, n_in = (int(v) for v in z[p + "meta"])
        yield dict(kind=str(z[p + "kind"]), t=t, rows=rows, n_in=n_in, raw=z[p + "raw"], x=z[p + "x"],
                   codes=z[p + "codes"], scales=z[p + "scales"], y=z[p + "y"], dots=z[p + "dots"],
                   xf=z[p + "xf"] if p + "xf" in z else None)


def test_golden_fixtures_present():
    assert sum(1 for _ in cases()) >= 40


def test_oracle_reproduces_golden():
    for c in cases():
        st, codes, scales = oracle.quant_act(c["x"])
        assert st == 0
        assert (codes == c["codes"]).all() and (scales == c["scales"]).all(), c["kind"]
        if c["xf"] is not None:
            st, cf, sf = oracle.quant_act_f32(c["xf"])
            assert st == 0 and (cf == c["codes"]).all() and (sf == c["scales"]).all()
        st, y = oracle.matvec_q8act(c["t"], c["raw"], c["rows"], c["n_in"], codes, scales)
        assert st == 0 and (y == c["y"]).all(), (c["kind"], c["t"], c["n_in"])
        if c["t"] not in (10, 11):  # the CPU baseline's fast cores cover the benchmarked families
            st, yf = oracle.matvec_q8act_fast(c["t"], c["raw"], c["rows"], c["n_in"], codes, scales, 2)
            assert st == 0 and (yf == c["y"]).all()
        rb = len(c["raw"]) // c["rows"]
        for r in range(c["rows"]):
            st, dots, _ = oracle.block_dots(c["t"], c["raw"][r * rb:(r + 1) * rb], c["n_in"], codes)
            assert st == 0 and (dots == c["dots"][r]).all()
