"""A fitted model: TabICL preprocessing plus the static context, predicting
from raw features (src/models/tabicl_v2/fitted.rs).

Fitting fits the preprocessing on the GPU, transforms the training rows into
each ensemble member's rows on the GPU, and builds the context from them.
Predicting transforms each chunk of raw rows straight into HBM (one kernel
per group and a member gather), runs the cached prediction on those device
rows, and aggregates the members' logits on the host. The fitted preprocessing
saves as IRPREP bytes and the context as IRCNTXT; `load_fitted` joins them
again (fitted.rs:318-352).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import context_file as cf
from . import hip, hipmem
from . import manifest as mf
from . import preprocess as pp
from .tabicl import Executor, StaticExecutor, aggregate_classifier_probabilities, summarize_regression


class FittedModel:
    """Preprocessing and context of one fit (FittedModel, fitted.rs:180-300)."""

    def __init__(self, executor: Executor, preprocessor: pp.Preprocessor, context: StaticExecutor):
        self.executor = executor
        self.preprocessor = preprocessor
        self.context = context

    # ---- fitting (Preprocessed::fit / with_training, Executor::build_fitted) ----

    @classmethod
    def fit(cls, executor: Executor, x, y, options: pp.PreprocessOptions | None = None,
            cache_dir=False) -> "FittedModel":
        """Fit on raw features x [rows, columns] and labels (classifier) or
        target values (regressor), then build the context on the GPU."""
        options = options or pp.PreprocessOptions()
        if executor.task == mf.CLASSIFIER:
            p = pp.Preprocessor.fit(options, x, y, executor.device)
        else:
            p = pp.Preprocessor.fit_regressor(options, x, y, executor.device)
        return cls._build(executor, p, x, y, cache_dir)

    @classmethod
    def _build(cls, executor: Executor, p: pp.Preprocessor, x, y, cache_dir) -> "FittedModel":
        if p.task != executor.task:
            raise ValueError(f"the preprocessing is for a {p.task}, but the model is a {executor.task}")
        rows, targets = training_inputs(p, x, y)
        context = executor.build_context(rows, targets, class_permutations=p.class_permutations,
                                         feature_permutations=p.feature_permutations, cache_dir=cache_dir)
        return cls(executor, p, context)

    # ---- prediction (FittedModel::predict_*, fitted.rs:205-275) ----

    def _chunks(self, x):
        """Yields (start, n, decoded outputs [B, n, width] in HBM) for raw rows
        x, in chunks of 8,192 rows transformed on the GPU into HBM."""
        x = np.asarray(x)
        if x.ndim != 2 or x.shape[0] == 0:
            raise ValueError("X must be a nonempty matrix of features")
        p = self.preprocessor
        p.attach(self.executor.device)
        b, h, width = p.member_count, p.n_features_out, self.executor.width
        q = x.shape[0]
        step = pp.PREDICT_CHUNK_ROWS
        rows_dev = hipmem.DeviceArray((b, min(step, q), h))
        logits_dev = hipmem.DeviceArray((b, min(step, q), width))
        flags = np.zeros(min(step, q), np.uint8)
        for start in range(0, q, step):
            chunk = x[start:start + step]
            n = chunk.shape[0]
            p.member_rows_device(chunk, rows_dev.ptr, chunk_rows=step)
            hip.check(hip.lib().irx_predictor_predict_device(
                self.context.handle, rows_dev.ptr, n, logits_dev.ptr,
                flags.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))))
            if flags[:n].any():
                raise ValueError("a row is the all-missing marker, which this backend does not predict")
            # The chunk's x and outputs are [B, n, *] from the start of the buffers.
            yield start, n, logits_dev

    def _logits(self, x) -> np.ndarray:
        """Every member's decoder outputs [B, Q, width] for raw rows x."""
        b, width = self.preprocessor.member_count, self.executor.width
        out = np.empty((b, np.asarray(x).shape[0], width), np.float32)
        for start, n, dev in self._chunks(x):
            out[:, start:start + n] = dev.to_host().reshape(-1)[: b * n * width].reshape(b, n, width)
        return out

    def predict_regression_outputs(self, x, output_types=("mean",), alphas=()) -> list[np.ndarray]:
        """Regression outputs (RegressionOutput, quantiles.rs:26-63) in the
        targets' units, summarized on the GPU chunk by chunk: the
        standardized values times the target scale plus its mean (unscale,
        fitted.rs:158-177); the variance scales by the square of the scale."""
        p = self.preprocessor
        if p.target_scale is None:
            raise ValueError("a classifier has no regression outputs")
        b, width = p.member_count, self.executor.width
        parts = [[] for _ in output_types]
        for start, n, dev in self._chunks(x):
            outs = summarize_regression(self.executor.device, dev.ptr, (b, n, width), output_types, alphas)
            for acc, o in zip(parts, outs):
                acc.append(o)
        m, s = p.target_scale
        result = []
        for name, acc in zip(output_types, parts):
            v = np.concatenate(acc).astype(np.float64)
            v = v * (s * s) if name == "variance" else v * s + m
            result.append(v.astype(np.float32))
        return result

    def predict_proba(self, x, temperature: float = 0.9, average_logits: bool = True) -> np.ndarray:
        """Class probabilities [Q, C] from raw rows (predict_probabilities)."""
        p = self.preprocessor
        if p.classes is None:
            raise ValueError("a regressor has no class probabilities")
        logits = self._logits(x)[:, :, : len(p.classes)]
        perms = np.asarray(p.class_permutations, dtype=np.int64)
        return aggregate_classifier_probabilities(logits, perms, temperature, average_logits)

    def predict(self, x, **kwargs):
        """Class labels (classifier) or mean predictions in target units (regressor)."""
        p = self.preprocessor
        if p.classes is not None:
            proba = self.predict_proba(x, **kwargs)
            return np.asarray(p.classes, dtype=object if p.label_kind == "text" else None)[proba.argmax(axis=1)]
        mean, _ = self.predict_quantiles(x)
        return mean

    def predict_quantiles(self, x, alphas=(0.05, 0.5, 0.95)) -> tuple[np.ndarray, np.ndarray]:
        """(mean [Q], quantiles [Q, len(alphas)]) in the targets' units: the
        standardized outputs times the target scale plus its mean (unscale,
        fitted.rs:158-177)."""
        p = self.preprocessor
        if p.target_scale is None:
            raise ValueError("a classifier has no regression outputs")
        mean, quantiles = self.predict_regression_outputs(x, ("mean", "quantiles"), alphas)
        return mean, quantiles

    # ---- persistence ----

    def preprocessor_bytes(self) -> bytes:
        """IRPREP bytes (FittedModel::preprocessor_bytes)."""
        return pp.encode_irprep(self.preprocessor, self.context.metadata.model_sha256)

    def context_bytes(self) -> bytes:
        import io

        sink = io.BytesIO()
        self.context.encode_context(sink)
        return sink.getvalue()

    @classmethod
    def load(cls, executor: Executor, preprocessor: bytes, context: bytes | None = None, training=None,
             cache_dir=False) -> "FittedModel":
        """Executor::load_fitted (fitted.rs:318-352): IRPREP bytes, and the
        IRCNTXT bytes or the training (x, y) to rebuild the context from."""
        sha, p = pp.decode_irprep(preprocessor)
        if sha.hex() != executor.source_sha256:
            raise ValueError(f"this {p.task} was fitted with checkpoint {sha.hex()}, not {executor.source_sha256}")
        p.attach(executor.device)
        if context is None:
            if training is None:
                raise ValueError("the training rows were not kept, so no context can be built")
            return cls._build(executor, p, training[0], training[1], cache_dir)
        st = executor.load_context_bytes(context)
        check_context(p, sha, st.metadata)
        return cls(executor, p, st)


def training_inputs(p: pp.Preprocessor, x, y) -> tuple[np.ndarray, np.ndarray]:
    """Each member's training rows [B, N, H] (transformed on the GPU, one
    batch) and targets [B, N]: class codes through the member's class order,
    or the standardized target values (Preprocessed::training_inputs,
    fitted.rs:103-131)."""
    rows = p.member_rows(x)
    if p.classes is not None:
        codes = p.encode_labels(y)
        targets = np.stack([np.asarray(order, np.float32)[codes] for order in p.class_permutations])
    else:
        m, s = p.target_scale
        scaled = ((np.asarray(y, np.float32).astype(np.float64) - m) / s).astype(np.float32)
        targets = np.tile(scaled, (p.member_count, 1))
    return rows, targets


def check_context(p: pp.Preprocessor, sha: bytes, meta: cf.Metadata) -> None:
    """check_context (fitted.rs:280-300): the context must be the one this
    preprocessing built."""
    classes = len(p.classes) if p.classes is not None else 0
    corders = np.asarray(p.class_permutations, dtype=np.uint64).reshape(-1)
    forders = np.asarray(p.feature_permutations, dtype=np.uint64).reshape(-1)
    if (meta.model_sha256 != sha or meta.ensemble_count != p.member_count
            or meta.feature_count != p.n_features_out or meta.class_count != classes
            or not np.array_equal(meta.class_permutations, corders)
            or not np.array_equal(meta.feature_permutations, forders)):
        raise ValueError("the context does not match its preprocessing (IRPREP)")
