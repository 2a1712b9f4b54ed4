"""Loading of the golden fixtures in tests/golden/ (numeric .npz only, no pickle)."""

from __future__ import annotations

from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def load_golden(name):
    """Load a golden case, regenerating workload inputs from their seed (SHA-256 checked)."""
    with np.load(GOLDEN / f"{name}.npz") as z:
        g = {key: z[key] for key in z.files}
    if "X" not in g:
        from skmetal_amd import _synth

        X, C0 = _synth.generate(str(g["workload"]), seed=int(g["seed"]), scale=float(g["scale"]))
        assert _synth.sha256(X) == str(g["sha256"]), "workload generator no longer reproduces the fixture input"
        np.testing.assert_array_equal(C0, g["C0"])
        g["X"] = X
    g["labels"] = g["labels"].astype(np.int32)
    return g
