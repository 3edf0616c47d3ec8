"""TabICL's numeric preprocessing with the statistics fitted and the rows
transformed on the GPU (src/models/tabicl_v2/preprocess.rs, the reference's
Rust port of TabICL 2.1.1's pipeline).

Host side, as in the reference: validation, the constant-feature mask, class
labels (scikit-learn's LabelEncoder), the ensemble (feature orders from the
Latin-square closed form, class shifts, normalization groups, all drawn from
CPython's `random.Random(random_state)` as TabICL draws them), and the IRPREP
bytes (src/format/preprocessor.rs). Device side, through the C ABI: every
kept feature's statistics at once (`irx_preprocess_fit`, f64) and each
member's FP32 rows (`irx_preprocessor_transform`).
"""

from __future__ import annotations

import ctypes
import hashlib
import random
import struct
from dataclasses import dataclass, field

import numpy as np

from . import hip

NONE, POWER = "none", "power"
METHOD_CODES = {NONE: 0, POWER: 1}
MAX_MEMBERS = 4096
CLASSES = range(2, 11)
LATIN_FEATURES = 4000  # above this, feature orders are random samples (preprocess.rs:29)
PREDICT_CHUNK_ROWS = 8192  # rows transformed per batch when predicting (fitted.rs:13)
STATISTICS = 9


@dataclass
class PreprocessOptions:
    """PreprocessOptions (preprocess.rs:73-96)."""

    n_estimators: int = 8
    random_state: int = 42
    norm_methods: tuple[str, ...] = (NONE, POWER)
    outlier_threshold: float = 4.0

    def validate(self) -> None:
        if not 1 <= self.n_estimators <= MAX_MEMBERS:
            raise ValueError(f"n_estimators must be in 1..={MAX_MEMBERS}")
        methods = list(self.norm_methods)
        if not methods or len(set(methods)) != len(methods) or any(m not in METHOD_CODES for m in methods):
            raise ValueError("norm_methods must be a nonempty list of unique methods ('none', 'power')")
        if not (np.isfinite(self.outlier_threshold) and self.outlier_threshold > 0):
            raise ValueError("outlier_threshold must be positive and finite")


# ---- class labels (src/preprocess/labels.rs) ----

LABEL_KINDS = {"int": 1, "float": 2, "bool": 3, "text": 4}


def label_kind(labels) -> str:
    arr = np.asarray(labels)
    if arr.dtype == np.bool_:
        return "bool"
    if np.issubdtype(arr.dtype, np.integer):
        return "int"
    if np.issubdtype(arr.dtype, np.floating):
        return "float"
    return "text"


def label_classes(labels) -> tuple[str, list]:
    """The sorted distinct labels and their kind (Labels::classes)."""
    kind = label_kind(labels)
    values = list(np.asarray(labels).tolist()) if kind != "text" else [str(v) for v in labels]
    if kind == "float" and any(v != v for v in values):
        raise ValueError("labels must not be NaN")
    if kind == "text":
        # Rust orders strings by their UTF-8 bytes, as Python orders code points.
        return kind, sorted(set(values))
    return kind, sorted(set(values))


def encode_labels(labels, kind: str, classes: list) -> np.ndarray:
    """Each label's class index (Labels::encode)."""
    if label_kind(labels) != kind:
        raise ValueError("y has a different label type than the training labels")
    index = {c: i for i, c in enumerate(classes)}
    values = [str(v) for v in labels] if kind == "text" else np.asarray(labels).tolist()
    try:
        return np.array([index[v] for v in values], dtype=np.int64)
    except KeyError:
        raise ValueError("y contains labels the training labels did not") from None


# ---- the ensemble (preprocess.rs:297-434) ----

def feature_orders(features: int, members: int, seed: int) -> list[list[int]]:
    """TabICL's Shuffler(method="latin") orders (FeatureShuffles): the rows of
    a Latin square whose first row is the features in drawn order and whose
    row r is that row rotated right by r, rows and columns shuffled; random
    samples above 4,000 features; the identity for one member."""
    if members == 1:
        return [list(range(features))]
    rng = random.Random(seed)
    indices = list(range(features))
    if features > LATIN_FEATURES:
        return [rng.sample(indices, features) for _ in range(members)]
    first = []
    while len(indices) > 1:
        first.append(indices.pop(rng._randbelow(len(indices))))
    first.extend(indices)
    rows = list(range(features))
    rng.shuffle(rows)
    cols = list(range(features))
    rng.shuffle(cols)
    n = features
    return [[first[(cols[i] + n - r) % n] for r in rows] for i in range(n)]


def ensemble(options: PreprocessOptions, features: int, classes: int | None):
    """EnsembleGenerator (preprocess.rs:374-434): the methods that make groups,
    and each member's group, feature order and class order."""
    members = options.n_estimators
    shuffles = feature_orders(features, members, options.random_state)
    if classes is None:
        class_orders = [[]]
    elif members == 1:
        class_orders = [list(range(classes))]
    else:
        class_orders = [[(c - shift) % classes for c in range(classes)] for shift in range(classes)]
    combinations = list(range(len(shuffles) * len(class_orders)))
    random.Random(options.random_state).shuffle(combinations)
    methods = list(options.norm_methods)
    selected = [(combinations[k // len(methods)], methods[k % len(methods)])
                for k in range(min(members, len(combinations) * len(methods)))]
    group_methods = [m for m in methods if any(name == m for _, name in selected)]
    groups, forders, corders = [], [], []
    for g, method in enumerate(group_methods):
        for combination, name in selected:
            if name == method:
                groups.append(g)
                forders.append(shuffles[combination // len(class_orders)])
                corders.append(class_orders[combination % len(class_orders)])
    return group_methods, groups, forders, corders


# ---- the fitted preprocessor ----

def _features(x) -> tuple[np.ndarray, int]:
    """A C-ordered [rows, columns] f32 or f64 matrix and whether it is f64."""
    x = np.asarray(x)
    if x.dtype != np.float32:
        x = np.ascontiguousarray(x, dtype=np.float64)
        return x, 1
    return np.ascontiguousarray(x), 0


def _check_matrix(x: np.ndarray, columns: int | None = None) -> int:
    if x.ndim != 2 or x.shape[1] == 0 or x.shape[0] == 0:
        raise ValueError("X must be a nonempty matrix of features")
    if columns is not None and x.shape[1] != columns:
        raise ValueError(f"X has {x.shape[1]} features; expected {columns}")
    if not np.all(np.isfinite(x)):
        raise ValueError("X must contain only finite values")
    return x.shape[0]


@dataclass
class Preprocessor:
    """Fitted TabICL preprocessing (Preprocessor, preprocess.rs:437-452). It
    keeps no training rows. `statistics` [groups, 9, kept] holds each group's
    mean, scale, minimum, maximum, lower, upper (and lambda, mean, scale of
    a power group)."""

    feature_mask: np.ndarray
    group_methods: list[str]
    statistics: np.ndarray
    member_groups: list[int]
    feature_permutations: list[list[int]]
    class_permutations: list[list[int]]
    label_kind: str | None = None
    classes: list | None = None
    target_scale: tuple[float, float] | None = None
    _device: object = field(default=None, repr=False, compare=False)
    _handle: object = field(default=None, repr=False, compare=False)

    # -- shape --
    @property
    def n_features_in(self) -> int:
        return len(self.feature_mask)

    @property
    def n_features_out(self) -> int:
        return int(np.count_nonzero(self.feature_mask))

    @property
    def member_count(self) -> int:
        return len(self.member_groups)

    @property
    def kept(self) -> list[int]:
        return [j for j, k in enumerate(self.feature_mask) if k]

    @property
    def task(self) -> str:
        return "classifier" if self.classes is not None else "regressor"

    @classmethod
    def fit(cls, options: PreprocessOptions, x, targets, device: hip.Device) -> "Preprocessor":
        """Preprocessor::fit (preprocess.rs:475-546): `targets` are class labels
        for a classifier, or the regressor's float values with `regression`."""
        return _fit(cls, options, x, targets, device, regression=False)

    @classmethod
    def fit_regressor(cls, options: PreprocessOptions, x, values, device: hip.Device) -> "Preprocessor":
        return _fit(cls, options, x, values, device, regression=True)

    def encode_labels(self, labels) -> np.ndarray:
        if self.classes is None:
            raise ValueError("a regressor has no classes")
        return encode_labels(labels, self.label_kind, self.classes)

    # -- device --
    def attach(self, device: hip.Device) -> None:
        """Upload the statistics and member orders (irx_preprocessor_new)."""
        if self._handle is not None and self._device is device:
            return
        self.close()
        kept = np.asarray(self.kept, dtype=np.uint32)
        methods = np.asarray([METHOD_CODES[m] for m in self.group_methods], dtype=np.int32)
        stats = np.ascontiguousarray(self.statistics, dtype=np.float64)
        groups = np.asarray(self.member_groups, dtype=np.uint32)
        orders = np.ascontiguousarray(np.asarray(self.feature_permutations, dtype=np.uint32).reshape(-1))
        handle = ctypes.c_void_p()
        hip.check(hip.lib().irx_preprocessor_new(
            device.handle, self.n_features_in, kept.ctypes.data, len(kept), methods.ctypes.data, len(methods),
            stats.ctypes.data, self.member_count, groups.ctypes.data, orders.ctypes.data, ctypes.byref(handle)))
        self._device, self._handle = device, handle.value

    def close(self) -> None:
        if self._handle:
            hip.lib().irx_preprocessor_free(self._handle)
        self._handle = None

    def __del__(self):
        self.close()

    def _transform(self, x, chunk_rows: int, members: bool, out_ptr=None) -> np.ndarray | None:
        if self._handle is None:
            raise ValueError("the preprocessor is not attached to a device (Preprocessor.attach)")
        x, f64 = _features(x)
        rows = _check_matrix(x, self.n_features_in)
        if out_ptr is not None:
            hip.check(hip.lib().irx_preprocessor_transform(self._handle, x.ctypes.data, f64, rows, chunk_rows,
                                                           1, out_ptr, 1))
            return None
        shape = (self.member_count if members else len(self.group_methods), rows, self.n_features_out)
        out = np.empty(shape, np.float32)
        hip.check(hip.lib().irx_preprocessor_transform(self._handle, x.ctypes.data, f64, rows, chunk_rows,
                                                       int(members), out.ctypes.data, 0))
        return out

    def transform(self, x, chunk_rows: int | None = None) -> np.ndarray:
        """Each group's FP32 rows [groups, rows, kept] (Preprocessor::transform,
        preprocess.rs:548-573), in batches of `chunk_rows` (default: one batch)."""
        x = np.asarray(x)
        return self._transform(x, chunk_rows or max(1, x.shape[0]), members=False)

    def member_rows(self, x, chunk_rows: int | None = None) -> np.ndarray:
        """Each member's feature-permuted rows [members, rows, kept]
        (transform + ensemble_rows, preprocess.rs:575-613)."""
        x = np.asarray(x)
        return self._transform(x, chunk_rows or max(1, x.shape[0]), members=True)

    def member_rows_device(self, x, out_ptr: int, chunk_rows: int = PREDICT_CHUNK_ROWS) -> None:
        """The same into device memory [members, rows, kept] at `out_ptr`."""
        self._transform(np.asarray(x), chunk_rows, members=True, out_ptr=out_ptr)

    def validate(self) -> None:
        """Preprocessor::validate (preprocess.rs:683-731), for bytes read from outside."""
        features = self.n_features_out
        groups = len(self.group_methods)
        classes = len(self.classes) if self.classes is not None else 0
        members = self.member_count

        def fail(msg):
            raise ValueError(f"preprocessor: {msg}")

        if features == 0:
            fail("no features are kept")
        if groups == 0 or len(set(self.group_methods)) != groups:
            fail("the normalization groups are invalid")
        if (not 1 <= members <= MAX_MEMBERS or len(self.feature_permutations) != members
                or len(self.class_permutations) != members or any(g >= groups for g in self.member_groups)
                or any(g not in self.member_groups for g in range(groups))):
            fail("the ensemble members are invalid")
        perm = lambda o, n: len(o) == n and sorted(o) == list(range(n))
        if (not all(perm(o, features) for o in self.feature_permutations)
                or not all(perm(o, classes) for o in self.class_permutations)):
            fail("a member's feature or class order is not a permutation")
        if self.classes is not None and not (len(self.classes) in CLASSES
                                             and all(a < b for a, b in zip(self.classes, self.classes[1:]))):
            fail("the classes are invalid")
        if self.classes is not None and self.target_scale is not None:
            fail("the target scale does not match the task")
        if self.classes is None:
            ts = self.target_scale
            if ts is None or not (np.isfinite(ts[0]) and np.isfinite(ts[1]) and ts[1] > 0):
                fail("the target scale does not match the task")
        for g, method in enumerate(self.group_methods):
            count = STATISTICS if method == POWER else 6
            if self.statistics.shape[2] != features or not np.all(np.isfinite(self.statistics[g, :count])):
                fail("a group's statistics are invalid")


def _fit(cls, options: PreprocessOptions, x, targets, device: hip.Device, regression: bool) -> Preprocessor:
    options.validate()
    x, f64 = _features(x)
    rows = _check_matrix(x)
    if len(targets) != rows:
        raise ValueError("X and y must have the same length")
    if rows < 2:
        raise ValueError("X and y must have at least two training rows")
    kind = classes = target_scale = None
    if not regression:
        kind, classes = label_classes(targets)
        if len(classes) not in CLASSES:
            raise ValueError("The classifier requires 2..10 classes")
    else:
        values = np.asarray(targets, dtype=np.float32).astype(np.float64)
        if not np.all(np.isfinite(values)):
            raise ValueError("y must contain only finite values")
        target_scale = _standard_scaler(values)
    mask = np.any(x[1:] != x[0], axis=0)
    kept = np.flatnonzero(mask).astype(np.uint32)
    if len(kept) == 0:
        raise ValueError("Training data must contain at least one nonconstant feature")
    group_methods, member_groups, forders, corders = ensemble(options, len(kept),
                                                              None if regression else len(classes))
    methods = np.asarray([METHOD_CODES[m] for m in group_methods], dtype=np.int32)
    stats = np.zeros((len(group_methods), STATISTICS, len(kept)), np.float64)
    hip.check(hip.lib().irx_preprocess_fit(device.handle, x.ctypes.data, f64, rows, x.shape[1], kept.ctypes.data,
                                           len(kept), methods.ctypes.data, len(methods),
                                           float(options.outlier_threshold), stats.ctypes.data))
    p = cls(mask.astype(bool), group_methods, stats, member_groups, forders, corders, kind, classes, target_scale)
    p.attach(device)
    return p


def _standard_scaler(values: np.ndarray) -> tuple[float, float]:
    """scale.rs standard_scaler, for the regressor's targets (host, f64)."""
    n = float(len(values))
    mean = float(np.sum(values) / n)
    d = values - mean
    correction, squares = float(np.sum(d)), float(np.sum(d * d))
    variance = (squares - correction * correction / n) / n
    eps = np.finfo(np.float64).eps
    bound = n * mean * eps
    constant = variance <= n * eps * variance + bound * bound
    return mean, (1.0 if constant else float(np.sqrt(variance)))


# ---- IRPREP (src/format/preprocessor.rs) ----

IRPREP_MAGIC = b"IRPREP\0\0"
IRPREP_VERSION = 1


def encode_irprep(p: Preprocessor, checkpoint_sha256: bytes) -> bytes:
    """The fitted preprocessing as IRPREP bytes (preprocessor.rs encode)."""
    if len(checkpoint_sha256) != 32:
        raise ValueError("checkpoint SHA-256 must be 32 bytes")
    out = bytearray(IRPREP_MAGIC)
    out += struct.pack("<I", IRPREP_VERSION) + checkpoint_sha256
    out += struct.pack("<Q", p.n_features_in) + bytes(int(bool(k)) for k in p.feature_mask)
    out += bytes([len(p.group_methods)]) + bytes(METHOD_CODES[m] for m in p.group_methods)
    out += struct.pack("<Q", p.member_count) + bytes(p.member_groups)
    for order in p.feature_permutations:
        out += struct.pack(f"<{len(order)}Q", *order)
    classes = len(p.classes) if p.classes is not None else 0
    out += struct.pack("<Q", classes)
    for order in p.class_permutations:
        out += struct.pack(f"<{len(order)}Q", *order)
    if p.classes is None:
        out += b"\0"
    else:
        out += bytes([LABEL_KINDS[p.label_kind]])
        if p.label_kind == "int":
            out += struct.pack(f"<{classes}q", *p.classes)
        elif p.label_kind == "float":
            out += struct.pack(f"<{classes}d", *p.classes)
        elif p.label_kind == "bool":
            out += bytes(int(bool(c)) for c in p.classes)
        else:
            for c in p.classes:
                raw = c.encode()
                out += struct.pack("<I", len(raw)) + raw
    if p.target_scale is not None:
        out += struct.pack("<2d", *p.target_scale)
    for g, method in enumerate(p.group_methods):
        count = STATISTICS if method == POWER else 6
        out += np.ascontiguousarray(p.statistics[g, :count], dtype="<f8").tobytes()
    return bytes(out) + hashlib.sha256(out).digest()


class _Reader:
    def __init__(self, data: bytes):
        self.data, self.pos = data, 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.data):
            raise ValueError("IRPREP is truncated")
        out = self.data[self.pos:self.pos + n]
        self.pos += n
        return out

    def u8(self) -> int:
        return self.take(1)[0]

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.take(8))[0]


def decode_irprep(data: bytes) -> tuple[bytes, Preprocessor]:
    """IRPREP bytes -> (checkpoint SHA-256, preprocessor), verified
    (preprocessor.rs decode)."""
    if len(data) < len(IRPREP_MAGIC) + 4 + 32 + 32:
        raise ValueError("IRPREP is truncated")
    body, digest = data[:-32], data[-32:]
    if hashlib.sha256(body).digest() != digest:
        raise ValueError("IRPREP checksum mismatch")
    r = _Reader(body)
    if r.take(8) != IRPREP_MAGIC:
        raise ValueError("not fitted preprocessing (IRPREP)")
    version = r.u32()
    if version != IRPREP_VERSION:
        raise ValueError(f"unsupported IRPREP version {version}; expected {IRPREP_VERSION}")
    sha = r.take(32)

    def flags(n):
        out = []
        for b in r.take(n):
            if b > 1:
                raise ValueError("IRPREP has an invalid flag")
            out.append(bool(b))
        return out

    mask = np.array(flags(r.u64()), dtype=bool)
    features = int(mask.sum())
    groups = []
    for b in r.take(r.u8()):
        if b > 1:
            raise ValueError("IRPREP has an invalid method")
        groups.append(POWER if b else NONE)
    members = r.u64()
    if members > MAX_MEMBERS:
        raise ValueError("IRPREP has too many members")
    member_groups = list(r.take(members))
    forders = [list(struct.unpack(f"<{features}Q", r.take(8 * features))) for _ in range(members)]
    classes = r.u64()
    if classes > 10:
        raise ValueError("IRPREP has too many classes")
    corders = [list(struct.unpack(f"<{classes}Q", r.take(8 * classes))) for _ in range(members)]
    kind_code = r.u8()
    kind = labels = target_scale = None
    if kind_code == 0:
        labels = None
    elif kind_code == 1:
        kind, labels = "int", list(struct.unpack(f"<{classes}q", r.take(8 * classes)))
    elif kind_code == 2:
        kind, labels = "float", list(struct.unpack(f"<{classes}d", r.take(8 * classes)))
    elif kind_code == 3:
        kind, labels = "bool", flags(classes)
    elif kind_code == 4:
        kind, labels = "text", []
        for _ in range(classes):
            try:
                labels.append(r.take(r.u32()).decode("utf-8"))
            except UnicodeDecodeError:
                raise ValueError("IRPREP has a label that is not UTF-8") from None
    else:
        raise ValueError("IRPREP has an invalid label kind")
    if (len(labels) if labels is not None else 0) != classes:
        raise ValueError("IRPREP has classes without labels")
    if labels is None:
        target_scale = struct.unpack("<2d", r.take(16))
    stats = np.zeros((len(groups), STATISTICS, features))
    for g, method in enumerate(groups):
        count = STATISTICS if method == POWER else 6
        stats[g, :count] = np.frombuffer(r.take(8 * count * features), dtype="<f8").reshape(count, features)
    if r.pos != len(body):
        raise ValueError("IRPREP has trailing bytes")
    p = Preprocessor(mask, groups, stats, member_groups, forders, corders, kind, labels,
                     tuple(target_scale) if target_scale is not None else None)
    p.validate()
    return sha, p
