"""scikit-learn-style estimators over the fitted model: TabICLClassifier and
TabICLRegressor with the reference drop-ins' preprocessing and aggregation
options (python/ironicl/classifier.py:78-170, regressor.py:60-140). The model
weights come as an Executor (weights resident on the GPU); checkpoint download,
the PyTorch path and memory planning options of the reference have no
counterpart here."""

from __future__ import annotations

from numbers import Integral, Real

import numpy as np

from . import preprocess as pp
from .fitted import FittedModel
from .tabicl import Executor


def _options(n_estimators, norm_methods, outlier_threshold, random_state) -> pp.PreprocessOptions:
    """The drop-ins' option checks (python/ironicl/base.py:252-258): an
    unseeded ensemble is refused rather than silently seeded, and the numbers
    must have the types the Rust side converts."""
    if random_state is None:
        raise NotImplementedError("random_state=None is not supported")
    for name, value, kind in (("n_estimators", n_estimators, Integral), ("random_state", random_state, Integral),
                              ("outlier_threshold", outlier_threshold, Real)):
        if isinstance(value, bool) or not isinstance(value, kind):
            raise ValueError(f"{name} must be a{'n integer' if kind is Integral else ' number'}, not {value!r}")
    if norm_methods is None:
        methods = (pp.NONE, pp.POWER)
    elif isinstance(norm_methods, str):
        methods = (norm_methods,)
    else:
        methods = tuple(norm_methods)
    return pp.PreprocessOptions(int(n_estimators), int(random_state), methods, float(outlier_threshold))


class TabICLClassifier:
    def __init__(self, executor: Executor, n_estimators: int = 8, norm_methods=None, outlier_threshold: float = 4.0,
                 softmax_temperature: float = 0.9, average_logits: bool = True, random_state: int | None = 42,
                 cache_dir=False):
        self.executor = executor
        self.n_estimators, self.norm_methods = n_estimators, norm_methods
        self.outlier_threshold, self.random_state = outlier_threshold, random_state
        self.softmax_temperature, self.average_logits = softmax_temperature, average_logits
        self.cache_dir = cache_dir

    def fit(self, X, y) -> "TabICLClassifier":
        opts = _options(self.n_estimators, self.norm_methods, self.outlier_threshold, self.random_state)
        self.model_ = FittedModel.fit(self.executor, X, y, opts, cache_dir=self.cache_dir)
        p = self.model_.preprocessor
        self.classes_ = np.asarray(p.classes, dtype=object if p.label_kind == "text" else None)
        self.n_features_in_ = p.n_features_in
        return self

    def predict_proba(self, X) -> np.ndarray:
        return self.model_.predict_proba(X, self.softmax_temperature, self.average_logits)

    def predict(self, X) -> np.ndarray:
        return self.classes_[self.predict_proba(X).argmax(axis=1)]


class TabICLRegressor:
    def __init__(self, executor: Executor, n_estimators: int = 8, norm_methods=None, outlier_threshold: float = 4.0,
                 random_state: int | None = 42, cache_dir=False):
        self.executor = executor
        self.n_estimators, self.norm_methods = n_estimators, norm_methods
        self.outlier_threshold, self.random_state = outlier_threshold, random_state
        self.cache_dir = cache_dir

    def fit(self, X, y) -> "TabICLRegressor":
        opts = _options(self.n_estimators, self.norm_methods, self.outlier_threshold, self.random_state)
        self.model_ = FittedModel.fit(self.executor, X, y, opts, cache_dir=self.cache_dir)
        self.n_features_in_ = self.model_.preprocessor.n_features_in
        return self

    def predict(self, X, output_type: str = "mean", alphas=None):
        """TabICLRegressor.predict's output types: "mean", "variance", "median"
        -> [Q]; "quantiles" -> [Q, len(alphas)] (alphas default 0.05, 0.5,
        0.95); "raw_quantiles" -> [Q, 999]; a list of names -> a dict of them."""
        alphas = (0.05, 0.5, 0.95) if alphas is None else tuple(alphas)
        names = [output_type] if isinstance(output_type, str) else list(output_type)
        outs = self.model_.predict_regression_outputs(X, tuple(names), alphas)
        return outs[0] if isinstance(output_type, str) else dict(zip(names, outs))
