"""Seeded random-init TabICLv2 weights and the synthetic workloads.

Everything here is deterministic and platform-independent: a counter-based
SplitMix64 stream, uniforms from its top 53 bits, normals by Box-Muller in
float64 rounded to float32. The C++ side never regenerates these; it receives
the arrays through the C ABI.

Weight initialisation (random-init weights of the official architecture):
  - Linear weights and biases (in/out projections, FFNs, decoder, y encoders,
    QASS MLPs, the 3->128 input): U(-1/sqrt(fan_in), +1/sqrt(fan_in)),
    PyTorch's ``nn.Linear`` default;
  - LayerNorm: weight 1 + U(-0.1, 0.1), bias U(-0.1, 0.1);
  - ``ind_vectors`` and ``cls_tokens``: N(0, 1);
  - ``rope.freqs[i] = 100000 ** (-i / 8)`` (docs/model.md: base 100,000).

Workloads follow the five benchmark configurations (train rows x features,
classes, test rows); see ``WORKLOADS``.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import manifest as mf

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

CLASSIFIER_WEIGHT_SEED = 20260212
REGRESSOR_WEIGHT_SEED = 20260213


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


class Stream:
    """Counter-based SplitMix64: value i of key k is mix(k + (i + 1) * golden)."""

    def __init__(self, key: int):
        with np.errstate(over="ignore"):
            self.key = _mix(np.array([key & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64))[0]
        self.counter = 0

    def bits(self, count: int) -> np.ndarray:
        i = np.arange(self.counter + 1, self.counter + 1 + count, dtype=np.uint64)
        self.counter += count
        with np.errstate(over="ignore"):
            return _mix(self.key + i * _GOLDEN)

    def uniform(self, count: int) -> np.ndarray:
        """Float64 uniforms in [0, 1)."""
        return (self.bits(count) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)

    def uniform_range(self, count: int, lo: float, hi: float) -> np.ndarray:
        return (lo + (hi - lo) * self.uniform(count)).astype(np.float32)

    def normal(self, count: int, std: float = 1.0) -> np.ndarray:
        u1 = self.uniform(count)
        u2 = self.uniform(count)
        r = np.sqrt(-2.0 * np.log1p(-u1))
        return (std * r * np.cos(2.0 * np.pi * u2)).astype(np.float32)

    def permutation(self, count: int) -> np.ndarray:
        return np.argsort(self.uniform(count), kind="stable")


def _key(seed: int, salt: int) -> int:
    return (seed * 0x100000001B3 + salt) & 0xFFFFFFFFFFFFFFFF


def random_weights(task: str, seed: int | None = None) -> dict[str, np.ndarray]:
    """Seeded random-init weights for every tensor of the official manifest."""
    if seed is None:
        seed = CLASSIFIER_WEIGHT_SEED if task == mf.CLASSIFIER else REGRESSOR_WEIGHT_SEED
    out: dict[str, np.ndarray] = {}
    names = mf.tensor_manifest(task)
    for index, (name, shape) in enumerate(names.items()):
        s = Stream(_key(seed, index + 1))
        count = int(np.prod(shape))
        if name.endswith("rope.freqs"):
            v = (100000.0 ** (-np.arange(8, dtype=np.float64) / 8.0)).astype(np.float32)
        elif name.endswith("ind_vectors") or name.endswith("cls_tokens"):
            v = s.normal(count)
        elif name.endswith("norm1.weight") or name.endswith("norm2.weight") or name.endswith("ln.weight"):
            v = (1.0 + s.uniform_range(count, -0.1, 0.1)).astype(np.float32)
        elif name.endswith("norm1.bias") or name.endswith("norm2.bias") or name.endswith("ln.bias"):
            v = s.uniform_range(count, -0.1, 0.1)
        else:
            if name.endswith(".weight") or name.endswith("_weight"):
                fan_in = shape[1]
            else:
                wname = name[: -len("bias")] + "weight"
                fan_in = names[wname][1]
            bound = 1.0 / np.sqrt(fan_in)
            v = s.uniform_range(count, -bound, bound)
        out[name] = np.ascontiguousarray(v.reshape(shape), dtype=np.float32)
    return out


@dataclass(frozen=True)
class Workload:
    name: str
    task: str
    ensembles: int
    train_rows: int
    features: int
    test_rows: int
    classes: int
    data_seed: int
    run_rows: int = 1024


# The benchmark configurations, by what they are (rows x features, classes).
WORKLOADS = {
    "clf-1k": Workload("clf-1k", mf.CLASSIFIER, 1, 1024, 54, 8, 7, 1),
    "clf-10k": Workload("clf-10k", mf.CLASSIFIER, 1, 10_000, 100, 1024, 10, 2),
    "clf-50k": Workload("clf-50k", mf.CLASSIFIER, 1, 50_000, 64, 4096, 10, 3, run_rows=512),
    "reg-20k": Workload("reg-20k", mf.REGRESSOR, 1, 20_000, 200, 2048, 0, 4),
    "clf-200k": Workload("clf-200k", mf.CLASSIFIER, 8, 200_000, 500, 16_384, 10, 5),
}


def _labels_cover(y: np.ndarray, classes: int) -> bool:
    return bool(np.all(np.bincount(y.astype(np.int64), minlength=classes)[:classes] > 0))


def workload_data(w: Workload, train_rows: int | None = None, test_rows: int | None = None,
                  features: int | None = None):
    """(x_train [B,N,H], y [B,N], x_test [B,Q,H], meta) for a workload.

    ``train_rows``/``test_rows``/``features`` shrink it for parity tests.
    Classifier labels are argmax of a seeded map and cover every class
    (reseeded until they do). Member e > 0 of an ensemble permutes features by a
    seeded shuffle and shifts classes by e, as the ensemble preprocessing does.
    """
    n = train_rows or w.train_rows
    q = test_rows or w.test_rows
    h = features or w.features
    b = w.ensembles
    s = Stream(_key(w.data_seed, 0xDA7A))
    st = Stream(_key(w.data_seed + 1000, 0xDA7A))

    def draw(stream: Stream, rows: int) -> np.ndarray:
        if w.task == mf.REGRESSOR:
            return stream.uniform_range(rows * h, -3.0, 3.0).reshape(rows, h)
        x = stream.normal(rows * h).reshape(rows, h)
        if w.name == "clf-10k":
            cols = Stream(_key(w.data_seed, 0xC01)).permutation(h)[: max(1, h // 5)]
            x[:, cols] = np.exp(x[:, cols])
        return x

    x = draw(s, n)
    xt = draw(st, q)
    meta: dict = {}
    attempt = 0
    while True:
        ls = Stream(_key(w.data_seed, 0x1AB + attempt))
        if w.task == mf.REGRESSOR:
            wl = ls.normal(h, std=np.sqrt(1.0 / h))
            idx = ls.permutation(h)[: min(20, h)]
            a = ls.uniform_range(len(idx), 0.5, 2.0)
            target = x.astype(np.float64) @ wl.astype(np.float64)
            target += np.sin(a[None, :] * x[:, idx]).sum(axis=1)
            target += ls.normal(n, std=0.1)
            mean, std = float(target.mean()), float(target.std())
            y = ((target - mean) / std).astype(np.float32)
            meta["y_mean"], meta["y_std"] = mean, std
            break
        c = w.classes
        if w.name == "clf-10k":
            w1 = ls.normal(h * 64).reshape(h, 64)
            w2 = ls.normal(64 * c).reshape(64, c)
            y = np.argmax(np.tanh(x @ w1) @ w2, axis=1)
        else:
            wm = ls.normal(h * c).reshape(h, c)
            y = np.argmax(x @ wm, axis=1)
        if _labels_cover(y, c):
            y = y.astype(np.float32)
            break
        attempt += 1
        if attempt == 100:
            raise ValueError(f"{w.name}: no seeded labeller covers all {c} classes at {h} features")
    xs, ys, xts, perms, fperms = [], [], [], [], []
    for e in range(b):
        fp = np.arange(h) if e == 0 else Stream(_key(w.data_seed, 0xFE0 + e)).permutation(h)
        xs.append(x[:, fp])
        xts.append(xt[:, fp])
        fperms.append(fp)
        if w.task == mf.CLASSIFIER:
            c = w.classes
            perm = (np.arange(c) + e) % c
            # Member e sees label perm[c] for true class c; aggregation reads
            # logits[perm[c]] back as class c.
            ys.append(perm[y.astype(np.int64)].astype(np.float32))
            perms.append(perm)
        else:
            ys.append(y)
    meta["class_permutations"] = np.array(perms, dtype=np.uint64) if perms else None
    meta["feature_permutations"] = np.array(fperms, dtype=np.uint64)
    return (np.ascontiguousarray(np.stack(xs), dtype=np.float32),
            np.ascontiguousarray(np.stack(ys), dtype=np.float32),
            np.ascontiguousarray(np.stack(xts), dtype=np.float32), meta)
