"""The transformer golden fixtures are consistent with themselves and with the seeded inputs (no GPU).

Each fixture (``tests/golden/transformer_<case>.npz``, written by ``tests/golden/make_transformer_golden.py``
with the CPU oracle) stores for every parameter a sample of its gradient, its norm and largest magnitude,
and the sum and norm of each row and column. These must agree with one another as the mathematics fixes
them: the row sums and the column sums add to the same total, the squared row norms, squared column norms
and squared full norm are one quantity, no sampled entry or line norm exceeds what the full norm and the
largest magnitude allow, and there is one line statistic per row and per column of the parameter's shape.
"""

import json
import os

import numpy as np
import pytest

from tests.golden import transformer_cases as TC

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("case", sorted(TC.CASES))
def test_fixture_statistics_agree(case):
    z = np.load(os.path.join(HERE, f"transformer_{case}.npz"))
    meta = json.loads(str(z["meta"]))
    cfg = TC.CASES[case]
    assert meta["config"] == cfg.__dict__
    model, _, weights, ids, _ = TC.setup(cfg)
    assert TC.input_digest(weights, ids) == meta["digest"]
    params = dict(model.named_parameters())
    assert meta["params"] == list(params)
    for name in meta["params"]:
        rows, cols = TC.as_rows(params[name].shape)
        rs, cs = (z[f"{p}sum/{name}"].astype(np.float64) for p in ("row", "col"))
        rn, cn = (z[f"{p}norm/{name}"].astype(np.float64) for p in ("row", "col"))
        norm, gmax = float(z[f"grad_norm/{name}"]), float(z[f"grad_max/{name}"])
        assert rs.shape == rn.shape == (rows,) and cs.shape == cn.shape == (cols,), name
        scale = np.abs(rs).sum() + np.abs(cs).sum() + 1e-30
        assert abs(rs.sum() - cs.sum()) <= 1e-5 * scale, name
        assert np.sqrt((rn * rn).sum()) == pytest.approx(norm, rel=1e-5), name
        assert np.sqrt((cn * cn).sum()) == pytest.approx(norm, rel=1e-5), name
        assert np.all(np.abs(rs) <= rn * np.sqrt(cols) * (1 + 1e-5)), name  # Cauchy-Schwarz on each row
        assert np.all(np.abs(cs) <= cn * np.sqrt(rows) * (1 + 1e-5)), name
        assert rn.max() <= gmax * np.sqrt(cols) * (1 + 1e-5) and cn.max() <= gmax * np.sqrt(rows) * (1 + 1e-5)
        g = z[f"grad/{name}"].astype(np.float64)
        assert np.abs(g).max() <= gmax * (1 + 1e-6) and gmax <= norm * (1 + 1e-6), name
        idx = z[f"idx/{name}"]
        assert idx.min() >= 0 and idx.max() < rows * cols
