"""Reading the model fixtures under tests/golden/models/ (written by
make_model_fixtures.py from the reference executor's outputs). Plain numpy:
loading a fixture runs nothing from the reference."""

from __future__ import annotations

from pathlib import Path

import numpy as np

DIR = Path(__file__).resolve().parent / "models"


def fingerprint(g, inputs: dict) -> np.ndarray:
    """float64 [input sum, input sum of squares, weight sum, weight count]."""
    x = np.concatenate([np.asarray(v, np.float64).ravel() for v in inputs.values()])
    ws = [np.asarray(v, np.float64).ravel() for v in g.initializers.values() if v.dtype == np.float32]
    w = np.concatenate(ws) if ws else np.zeros(1)
    return np.array([x.sum(), np.square(x).sum(), w.sum(), float(w.size)])


def load(name: str) -> dict[str, np.ndarray]:
    """The fixture's arrays: out<i>_<tensor> for each graph output, and the
    fingerprint of the graph and input it was made from."""
    with np.load(DIR / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def outputs(name: str) -> list[np.ndarray]:
    """The fixture's graph outputs, in graph order."""
    arrays = load(name)
    keys = sorted((k for k in arrays if k.startswith("out")), key=lambda k: int(k[3:].split("_")[0]))
    return [arrays[k] for k in keys]


def matches(name: str, g, inputs: dict) -> bool:
    """True when `g` and `inputs` are what the fixture was made from."""
    return bool(np.allclose(fingerprint(g, inputs), load(name)["fingerprint"], rtol=1e-12, atol=0))
