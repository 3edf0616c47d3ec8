"""Host side of the ROCm backend: the reference's Executor / StaticExecutor
surface over the C ABI.

This mirrors how src/models/tabicl_v2/cpu.rs drives its CUDA backend
(``build_tensors_cuda`` cpu.rs:737-804, ``with_cuda`` cpu.rs:1855-1910,
``predict_logits`` cpu.rs:2057-2108): the host computes the QASSMax base
scales and the column stage's inducing queries, hands every array to
``irx_build`` / ``irx_predictor_*`` and post-processes logits (probability
aggregation, regression quantiles). The label embeddings, which the
reference's host computes, are computed by the device from the targets
(``Executor.device_labels``).

Nothing here computes the model on the CPU: rows the device flags for the
CPU path (a grouped all-missing -100 triple) come back as NaN logits and are
listed in ``Prediction.cpu_rows`` for the caller's own CPU path.
"""

from __future__ import annotations

import concurrent.futures
import ctypes
import hashlib
import math
import os
from dataclasses import dataclass, field

import numpy as np

from . import context_file as cf
from . import hip
from . import manifest as mf

_erf = np.frompyfunc(math.erf, 1, 1)

# The optimize levels this backend builds and predicts at (Precision::for_optimize,
# cuda/mod.rs:82-92): "safe" all FP32; "auto" an FP16 ICL cache with split-FP16
# attention products; "fast" the same FP16 context, resident as an FP8 cache
# read with single FP16 products.
PRECISION = {"safe": hip.PRECISION_FP32, "auto": hip.PRECISION_SPLIT, "fast": hip.PRECISION_HALF}


def _precision(optimize: str) -> int:
    if optimize not in PRECISION:
        raise ValueError(f"optimize must be one of {sorted(PRECISION)} on this backend, not {optimize!r}")
    return PRECISION[optimize]


def _gelu64(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + _erf(x / math.sqrt(2.0)).astype(np.float64))


def _layer_norm64(x: np.ndarray, w: np.ndarray, b: np.ndarray | None) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + 1e-5) * w
    return y + b if b is not None else y


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def validate_labels(y: np.ndarray, b: int, n: int) -> int:
    """Class count of [B, N] labels: contiguous 0..C-1 with C in 2..=10 and the
    same C for every estimator (validate_labels, cpu.rs:4717-4740)."""
    classes = None
    for e in range(b):
        lab = y[e]
        if not np.all((lab >= 0) & (lab <= 9) & (lab == np.floor(lab))):
            raise ValueError("labels must be integers in 0..=9")
        present = np.zeros(10, bool)
        present[lab.astype(np.int64)] = True
        c = 0
        while c < 10 and present[c]:
            c += 1
        if not 2 <= c <= 10 or present[c:].any():
            raise ValueError("each ensemble's labels must be contiguous 0..C-1 with C in 2..=10")
        if classes is not None and classes != c:
            raise ValueError("all ensembles must have the same class count")
        classes = c
    return int(classes)


@dataclass
class Prediction:
    """Decoder outputs [B, Q, outputs]; rows in ``cpu_rows`` hold NaN."""
    logits: np.ndarray
    cpu_rows: list[int] = field(default_factory=list)


class Executor:
    """An official TabICLv2 model with its weights resident on the GPU
    (Executor, cpu.rs:290-296; ModelWeights::new, cuda/weights.rs:299)."""

    # Builds hand the device the [B, N] targets, which it embeds through its
    # y_encoder weights (irx_build_inputs.targets). False: the host computes
    # the [B, N, 128] and [B, N, 512] embeddings and uploads them, as the
    # reference's BuildInputs carry them (the two give the same bits).
    device_labels = True

    def __init__(self, task: str, weights: dict[str, np.ndarray], device: hip.Device | None = None,
                 source_sha256: str | None = None):
        """`source_sha256` (64 hex digits) is the source checkpoint's SHA-256
        the model artifact records (ModelSummary::source_sha256), which
        context identities and IRCNTXT files carry. Without one, the SHA-256
        of the weights themselves stands in (`weights_sha256`)."""
        if task not in (mf.CLASSIFIER, mf.REGRESSOR):
            raise ValueError(f"unknown task {task!r}")
        self.task = task
        self.weights = {k: _f32(v) for k, v in weights.items()}
        self._constants: dict[int, tuple] = {}
        self.width = mf.decoder_width(task)
        if source_sha256 is None:
            source_sha256 = weights_sha256(task, self.weights)
        if len(source_sha256) != 64 or any(c not in "0123456789abcdef" for c in source_sha256):
            raise ValueError("source_sha256 must be 64 lowercase hex digits")
        self.source_sha256 = source_sha256
        self.device = device if device is not None else hip.Device(0)

        @hip.LOOKUP
        def lookup(_user, name, data, length):
            arr = self.weights.get(name.decode())
            if arr is None:
                return 1
            data[0] = arr.ctypes.data_as(hip._CF)
            length[0] = arr.size
            return 0

        handle = ctypes.c_void_p()
        t = hip.TASK_CLASSIFIER if task == mf.CLASSIFIER else hip.TASK_REGRESSOR
        hip.check(hip.lib().irx_weights_upload(self.device.handle, t, lookup, None, ctypes.byref(handle)))
        self.handle = handle.value

    @classmethod
    def from_model_file(cls, path, device: hip.Device | None = None) -> "Executor":
        """Weights from an IRMODEL artifact (ModelArtifact::load, src/format/model.rs:225-250;
        an official profile only), uploaded through irx_weights_upload; the
        artifact's source SHA-256 becomes the model identity contexts carry."""
        from . import model_file

        artifact = model_file.load(path)
        executor = cls(artifact.task, artifact.tensors, device, source_sha256=artifact.source_sha256)
        executor.artifact = artifact.summary
        return executor

    def __del__(self):
        h = getattr(self, "handle", None)
        if h:
            hip.lib().irx_weights_release(h)
            self.handle = None

    def tensor(self, name: str) -> np.ndarray:
        return self.weights[name]

    def budget(self, device_limit: int = 0) -> int:
        n = ctypes.c_size_t()
        hip.check(hip.lib().irx_weights_budget(self.handle, device_limit, ctypes.byref(n)))
        return n.value

    # ---- host preparations the build and predictor take (cpu.rs:573-599, 763-771) ----

    def target_embeddings(self, prefix: str, y: np.ndarray, width: int, out: np.ndarray | None = None) -> np.ndarray:
        """[N, width] label embeddings (target_embeddings, cpu.rs:1658-1680):
        weight[:, class] + bias for the classifier (one f32 sum per class,
        gathered by row), target * weight + bias for the regressor (two f32
        roundings, as the reference's loop)."""
        w = self.tensor(f"{prefix}.y_encoder.weight")
        b = self.tensor(f"{prefix}.y_encoder.bias")
        if out is None:
            out = np.empty((y.shape[0], width), np.float32)
        if self.task == mf.CLASSIFIER:
            table = _f32(w.T + b[None, :])  # [classes, width]
            # Labels are validated to 0..classes-1 before a build; "clip" lets
            # take write into `out` unbuffered.
            np.take(table, y.astype(np.intp), axis=0, out=out, mode="clip")
        else:
            np.multiply.outer(y.astype(np.float32), _f32(w[:, 0]), out=out)
            out += _f32(b)
        return out

    def label_embeddings(self, y: np.ndarray):
        """Column-stage [B, N, 128] and ICL-stage [B, N, 512] label embeddings."""
        b, n = y.shape
        col = np.empty((b, n, 128), np.float32)
        icl = np.empty((b, n, 512), np.float32)
        for e in range(b):
            self.target_embeddings("col_embedder", y[e], 128, col[e])
            self.target_embeddings("icl_predictor", y[e], 512, icl[e])
        return col, icl

    def qass_base_scale(self, prefix: str, source: int) -> np.ndarray:
        """base = W2 gelu(w1 ln(max(source,1)) + b1) + b2 in the reference's FP32
        arithmetic (qass_base_scale, cpu.rs:3768-3791): ln of the count rounded
        to f32, w1 * ln + b1 as one fused multiply-add, the GELU in f32, and
        the affine as a bias-initialized chain of fused multiply-adds
        (affine_f32, reference.rs:83-120). A large w1 makes the scale
        sensitive to the count, so its rounding is the reference's, not a
        float64 one's."""
        n = lambda part: self.tensor(f"{prefix}.ssmax_layer.{part}")
        log_source = np.float32(math.log(max(source, 1)))
        w1 = n("base_mlp.0.weight")[:, 0].astype(np.float64)
        # A product of two f32 values is exact in f64, so one rounding to f32
        # after the add is the fused multiply-add (up to a rare double rounding).
        value = (w1 * np.float64(log_source) + n("base_mlp.0.bias").astype(np.float64)).astype(np.float32)
        hidden = (np.float32(0.5) * value *
                  (np.float32(1.0) + _erf(value / np.float32(math.sqrt(2.0))).astype(np.float32))).astype(np.float32)
        w2 = n("base_mlp.2.weight").astype(np.float64)
        acc = n("base_mlp.2.bias").astype(np.float32)
        for k in range(hidden.shape[0]):
            acc = (acc.astype(np.float64) + np.float64(hidden[k]) * w2[:, k]).astype(np.float32)
        return _f32(acc)

    def icl_base_scales(self, n: int) -> list[np.ndarray]:
        return [self.qass_base_scale(f"icl_predictor.tf_icl.blocks.{b}.attn", n) for b in range(12)]

    def inducing_queries(self, n: int) -> list[np.ndarray]:
        """Each column block's inducing points as multihead_attn1 queries: norm1,
        the query projection and QASSMax for n sources, tokens [128, 128]
        (query_heads, cpu.rs:1421-1467; qassmax_f32, reference.rs:335-430)."""
        out = []
        for blk in range(3):
            p = f"col_embedder.tf_col.blocks.{blk}"
            a = f"{p}.multihead_attn1"
            ind = self.tensor(f"{p}.ind_vectors")
            norm = _layer_norm64(ind, self.tensor(f"{a}.norm1.weight"), self.weights.get(f"{a}.norm1.bias"))
            w = self.tensor(f"{a}.attn.in_proj_weight")[:128].astype(np.float64)
            bq = self.tensor(f"{a}.attn.in_proj_bias")[:128]
            q = norm @ w.T + bq                       # [128 rows, 128]
            qh = q.reshape(128, 8, 16)                # row, head, d
            s = lambda part: self.tensor(f"{a}.attn.ssmax_layer.{part}").astype(np.float64)
            base = self.qass_base_scale(f"{a}.attn", n).astype(np.float64).reshape(8, 16)
            hidden = _gelu64(qh @ s("query_mlp.0.weight").T + s("query_mlp.0.bias"))
            gate = hidden @ s("query_mlp.2.weight").T + s("query_mlp.2.bias")
            gated = qh * base[None, :, :] * (1.0 + np.tanh(gate))
            out.append(_f32(gated.reshape(128, 128)))
        return out

    def _row_count_constants(self, n: int):
        """inducing_queries(n) and icl_base_scales(n): functions of the weights
        and the train-row count only, kept for the last few counts (their
        float64 GELU runs libm's erf per element)."""
        hit = self._constants.get(n)
        if hit is None:
            hit = (self.inducing_queries(n), self.icl_base_scales(n))
            if len(self._constants) >= 8:
                self._constants.pop(next(iter(self._constants)))
            self._constants[n] = hit
        return hit

    def rope_frequencies(self) -> np.ndarray:
        return self.tensor("row_interactor.tf_row.rope.freqs")

    def cls_tokens(self) -> np.ndarray:
        return self.tensor("row_interactor.cls_tokens")

    # ---- build (build_context / build_tensors_cuda, cpu.rs:627-804) ----

    def context_metadata(self, x: np.ndarray, y_train: np.ndarray, class_permutations=None,
                         feature_permutations=None, optimize: str = "safe") -> cf.Metadata:
        """Validate a context's inputs and describe it, with its cache identity
        (context_metadata, cpu.rs:809-869). Permutations default to the
        identity: class [B, C] (classifier) and feature [B, H]."""
        meta, x, y_train = self._unhashed_metadata(x, y_train, class_permutations, feature_permutations)
        meta.context_sha256 = cf.context_identity(self.source_sha256, optimize, x, y_train,
                                                  meta.class_permutations, meta.feature_permutations)
        try:
            cf.validate_metadata(meta)
        except cf.ContextError as e:
            raise ValueError(str(e)) from None
        return meta

    def _unhashed_metadata(self, x, y_train, class_permutations, feature_permutations):
        """context_metadata's checks and description with a placeholder
        identity; also the f32 inputs the identity hashes."""
        x = _f32(x)
        y_train = _f32(y_train)
        if x.ndim != 3 or y_train.shape != x.shape[:2] or min(x.shape) == 0:
            raise ValueError("context needs nonempty x[B, N, H] and y_train[B, N]")
        b, n, h = x.shape
        classes = validate_labels(y_train, b, n) if self.task == mf.CLASSIFIER else 0
        if self.task == mf.REGRESSOR and not np.all(np.isfinite(y_train)):
            raise ValueError("regression targets must be finite")
        cperm = (np.asarray(class_permutations, dtype=np.uint64).reshape(-1) if class_permutations is not None
                 else np.tile(np.arange(classes, dtype=np.uint64), b))
        fperm = (np.asarray(feature_permutations, dtype=np.uint64).reshape(-1) if feature_permutations is not None
                 else np.tile(np.arange(h, dtype=np.uint64), b))
        meta = cf.Metadata(bytes.fromhex(self.source_sha256), b"\1" * 32, b, n, h, classes, cperm, fperm)
        try:
            cf.validate_metadata(meta)
        except cf.ContextError as e:
            raise ValueError(str(e)) from None
        return meta, x, y_train

    def build_context(self, x: np.ndarray, y_train: np.ndarray, class_permutations=None,
                      feature_permutations=None, download: bool = False, progress=None,
                      device_limit: int = 0, cache_dir=False, optimize: str = "safe") -> "StaticExecutor":
        """Build the static context of x [B, N, H], y_train [B, N] on the GPU and
        keep it resident (Executor::build_context, cpu.rs:600-673). With
        ``download``, also copy every cache tensor to the host
        (``StaticExecutor.context``).

        ``cache_dir`` (None/True: the default cache directory, False: none, or
        a path): load the context from ``<identity>.irctx`` there when that
        file holds exactly this context, else build it and write it there.
        A missing, invalid or mismatched entry is rebuilt; a failed write
        leaves the context in HBM only (cpu.rs:645-672). ``optimize`` is "safe"
        (all FP32), "auto" (an FP16 ICL cache read by split-FP16 attention) or
        "fast" (the FP16 context kept on the host, its ICL cache resident as
        FP8 with per-dim scales, read with single FP16 products)."""
        precision = _precision(optimize)
        directory = cf.resolve_cache_dir(cache_dir)
        if directory is None:
            # With no cache to look up, the identity (SHA-256 over x and
            # y_train) is only kept with the context: hash it on a host thread
            # while the GPU builds.
            meta, xf, yf = self._unhashed_metadata(x, y_train, class_permutations, feature_permutations)
            with concurrent.futures.ThreadPoolExecutor(1) as pool:
                identity = pool.submit(cf.context_identity, self.source_sha256, optimize, xf, yf,
                                       meta.class_permutations, meta.feature_permutations)
                executor = self._build(xf, yf, meta, download, progress, device_limit, precision)
                meta.context_sha256 = identity.result()
            return executor
        meta = self.context_metadata(x, y_train, class_permutations, feature_permutations, optimize)
        path = cf.cache_path(directory, meta)
        cached = cf.read_cached(path, meta)
        if cached is not None:
            try:
                cf.validate_for_model(cached, self.source_sha256, self.task)
            except cf.ContextError:
                cached = None
        if cached is not None:
            try:
                os.utime(path)  # the entry's last use, for clear_cache
            except OSError:
                pass
            try:
                return self._attach(cached, optimize)
            except cf.ContextError:
                pass  # stored at another precision: rebuilt below
        executor = self._build(_f32(x), _f32(y_train), meta, download, progress, device_limit, precision)
        # Caching is best effort: a context that cannot be written is still returned.
        try:
            directory.mkdir(parents=True, exist_ok=True)
            executor.save_context(path)
        except (OSError, ValueError):
            pass
        return executor

    def _build(self, x, y_train, meta: cf.Metadata, download: bool, progress, device_limit: int,
               precision: int = hip.PRECISION_FP32) -> "StaticExecutor":
        b, n, h = x.shape
        ind_q, bases = self._row_count_constants(n)
        freqs, cls = self.rope_frequencies(), self.cls_tokens()
        inp = hip.BuildInputs()
        inp.shape = hip.Shape(b, h, n, self.width)
        inp.x = hip.fptr(x)
        if self.device_labels:
            # The device embeds the targets through its y_encoder weights.
            targets = np.ascontiguousarray(y_train, np.float32)
            inp.targets = hip.fptr(targets)
        else:
            col_labels, icl_labels = self.label_embeddings(y_train)
            inp.column_labels, inp.icl_labels = hip.fptr(col_labels), hip.fptr(icl_labels)
        for i in range(3):
            inp.inducing_queries[i] = hip.fptr(ind_q[i])
        for i in range(12):
            inp.base_scales[i] = hip.fptr(bases[i])
        inp.rope_frequencies, inp.cls_tokens = hip.fptr(freqs), hip.fptr(cls)
        inp.budget = self.budget(device_limit)
        cb = _progress(progress)
        inp.progress = cb
        out = hip.BuildOutputs()
        context = None
        if download:
            ck = [np.zeros((b, h + 4, 8, 128, 16), np.float32) for _ in range(3)]
            cv = [np.zeros_like(ck[0]) for _ in range(3)]
            icl_dtype = np.float32 if precision == hip.PRECISION_FP32 else np.float16
            ik = [np.zeros((b, 8, n, 64), icl_dtype) for _ in range(12)]
            iv = [np.zeros_like(ik[0]) for _ in range(12)]
            for i in range(3):
                out.column_keys[i], out.column_values[i] = hip.fptr(ck[i]), hip.fptr(cv[i])
            for i in range(12):
                out.icl_keys[i], out.icl_values[i] = hip.cache_ptr(ik[i]), hip.cache_ptr(iv[i])
            context = (ck, cv, ik, iv)
        keep = ctypes.c_void_p()
        hip.check(hip.lib().irx_build(self.handle, precision, ctypes.byref(inp), ctypes.byref(out),
                                      ctypes.byref(keep)))
        return StaticExecutor(self, (b, n, h), meta.class_count, meta.class_permutations,
                              meta.feature_permutations, built=keep.value, context=context, base_scales=bases,
                              metadata=meta, precision=precision)

    def _attach(self, context: cf.ContextFile, optimize: str | None = None) -> "StaticExecutor":
        """Upload a verified context for prediction (with_executor / with_cuda,
        cpu.rs:1745-1910). Its ICL storage decides the precision: FP32 caches
        predict at "safe", FP16 caches at "auto" (the default) or "fast" (the
        file does not record which: the caller's level does); asking an FP32
        context for "auto"/"fast" or an FP16 one for "safe" is an error (the
        reference's CUDA path would leave such a context on its CPU, which
        this backend does not have)."""
        meta = context.metadata
        b, n, _ = meta.shape
        icl = {context.tensor(f"icl.{i}.{kind}").dtype for i in range(12) for kind in ("key", "value")}
        cols = {context.tensor(f"column.{i}.{kind}").dtype for i in range(3) for kind in ("key", "value")}
        if cols != {np.dtype("<f4")} or len(icl) != 1:
            raise cf.ContextError("the context's column caches must be FP32 and its ICL caches of one type")
        levels = ("auto", "fast") if icl == {np.dtype("<f2")} else ("safe",)
        if optimize is not None and optimize not in levels:
            raise cf.ContextError(f"the context stores its ICL cache for optimize={levels[0]!r}, not {optimize!r}")
        stored = optimize if optimize is not None else levels[0]
        return StaticExecutor(self, meta.shape, meta.class_count, meta.class_permutations,
                              meta.feature_permutations, built=None, context=context.host_tensors(),
                              base_scales=self.icl_base_scales(n), metadata=meta, keep_alive=context,
                              precision=_precision(stored))

    def predict_input_bundle(self, bundle) -> Prediction:
        """Uncached prediction of an IRINPUT bundle (Executor::predict_logits,
        cpu.rs:970-1030): each estimator's first N of its T rows are the
        training rows, the other T - N are predicted; logits [B, T - N, C]."""
        if self.task != mf.CLASSIFIER:
            raise ValueError("IRINPUT bundles carry classifier inputs")
        b, t, h, n = bundle.shape
        ctx = self.build_context(np.ascontiguousarray(bundle.x[:, :n]), bundle.y_train)
        return ctx.predict_logits(np.ascontiguousarray(bundle.x[:, n:]))

    def load_context(self, path, optimize: str | None = None) -> "StaticExecutor":
        """Load a persisted IRCNTXT context, verify it against this model and
        upload it to HBM (Executor::load_context, cpu.rs:397-406)."""
        context = cf.read(path)
        cf.validate_for_model(context, self.source_sha256, self.task)
        return self._attach(context, optimize)

    def load_context_bytes(self, data: bytes, optimize: str | None = None) -> "StaticExecutor":
        """The same from the bytes ``StaticExecutor.encode_context`` wrote
        (Executor::load_context_bytes, cpu.rs:415-424)."""
        context = cf.from_bytes(data)
        cf.validate_for_model(context, self.source_sha256, self.task)
        return self._attach(context, optimize)

    def load_context_tensors(self, context, shape, classes: int, class_permutations=None,
                             feature_permutations=None, device_limit: int = 0) -> "StaticExecutor":
        """Upload host context tensors (column K/V [B,H+4,8,128,16] x 3 each, ICL
        K/V [B,8,N,64] x 12 each) for prediction, without a file. ``device_limit``
        (bytes, 0 = none) caps the device memory the model may use
        (ModelWeights::budget, cuda/weights.rs:286-292): the predictor takes one
        stream and halves its passes until its workspace fits beside the caches."""
        b, n, h = shape
        return StaticExecutor(self, (b, n, h), classes, class_permutations, feature_permutations,
                              built=None, context=context, base_scales=self.icl_base_scales(n),
                              device_limit=device_limit)


def weights_sha256(task: str, weights: dict[str, np.ndarray]) -> str:
    """A model identity from the weights themselves: SHA-256 over the task and,
    in the official manifest's order, each tensor's name, shape and FP32
    bytes. It stands in for a source checkpoint's SHA-256 when there is none
    (random-init weights)."""
    digest = hashlib.sha256(f"ironicl-weights\0{task}\0".encode())
    for name, shape in mf.tensor_manifest(task).items():
        arr = weights.get(name)
        if arr is None:
            continue
        arr = np.ascontiguousarray(arr, dtype="<f4")
        digest.update(name.encode() + b"\0" + np.asarray(arr.shape, dtype="<u8").tobytes())
        digest.update(memoryview(arr).cast("B"))
    return digest.hexdigest()


def _progress(fn):
    if fn is None:
        return hip.PROGRESS()

    @hip.PROGRESS
    def cb(_user, stage, done, total):
        try:
            fn(stage, done, total)
            return 0
        except Exception:
            return 1

    return cb


class StaticExecutor:
    """A context resident on the GPU and its predictor (StaticExecutor, cpu.rs:313-326;
    Predictor, cuda/predictor.rs:93-271)."""

    def __init__(self, executor: Executor, shape, classes: int, class_permutations, feature_permutations,
                 built, context, base_scales, metadata: cf.Metadata | None = None, keep_alive=None,
                 precision: int = hip.PRECISION_FP32, device_limit: int = 0):
        self.executor = executor
        self.shape = shape
        self.classes = classes
        self.metadata = metadata
        self.precision = precision
        self._keep_alive = keep_alive
        b = shape[0]
        self.class_permutations = (np.asarray(class_permutations, dtype=np.uint64).reshape(b, -1)
                                   if class_permutations is not None
                                   else (np.tile(np.arange(classes, dtype=np.uint64), (b, 1)) if classes else None))
        self.feature_permutations = feature_permutations
        self.context = context
        b, n, h = shape
        ctx = hip.ContextTensors()
        ctx.shape = hip.Shape(b, h, n, executor.width)
        self._bases = [_f32(s) for s in base_scales]
        for i in range(12):
            ctx.base_scales[i] = hip.fptr(self._bases[i])
        ctx.rope_frequencies = hip.fptr(executor.rope_frequencies())
        ctx.cls_tokens = hip.fptr(executor.cls_tokens())
        ctx.budget = executor.budget(device_limit)
        keep_alive = []
        if built is None:
            icl_dtype = np.float32 if precision == hip.PRECISION_FP32 else np.float16
            ck, cv = [[_f32(t) for t in part] for part in context[:2]]
            ik, iv = [[np.ascontiguousarray(t, dtype=icl_dtype) for t in part] for part in context[2:]]
            keep_alive = [ck, cv, ik, iv]
            for i in range(3):
                ctx.column_keys[i], ctx.column_values[i] = hip.fptr(ck[i]), hip.fptr(cv[i])

            @hip.ICL_SOURCE
            def source(_user, block, keys, values):
                if block >= 12:
                    return 1
                keys[0] = ik[block].ctypes.data_as(hip._CF)
                values[0] = iv[block].ctypes.data_as(hip._CF)
                return 0

            ctx.icl = source
            keep_alive.append(source)
        handle = ctypes.c_void_p()
        hip.check(hip.lib().irx_predictor_new(executor.handle, precision, ctypes.byref(ctx), built,
                                              ctypes.byref(handle)))
        self.handle = handle.value

    def __del__(self):
        h = getattr(self, "handle", None)
        if h:
            hip.lib().irx_predictor_free(h)
            self.handle = None

    def device(self) -> str:
        return "rocm"

    def streamed(self) -> bool:
        return bool(hip.lib().irx_predictor_streamed(self.handle))

    def pass_rows(self) -> int:
        return int(hip.lib().irx_predictor_pass_rows(self.handle))

    def set_pass_rows(self, rows: int) -> None:
        hip.check(hip.lib().irx_predictor_set_pass_rows(self.handle, rows))

    def set_graphs(self, enable: bool) -> None:
        """Replay prediction passes from HIP graphs (the default) or launch
        their kernels one by one; results are identical."""
        hip.check(hip.lib().irx_predictor_set_graphs(self.handle, int(bool(enable))))

    def set_streams(self, streams: int) -> None:
        """Passes rotate over `streams` (1 to 4) HIP streams; results are identical."""
        hip.check(hip.lib().irx_predictor_set_streams(self.handle, streams))

    def outputs(self) -> int:
        return self.classes if self.classes else self.executor.width

    # ---- persistence (StaticExecutor::save_context / encode_context, cpu.rs:1716-1742) ----

    def _tensor_source(self):
        """Values of each context tensor, from the host copy when there is one,
        otherwise streamed out of HBM (irx_predictor_read_context; a "fast"
        build keeps its FP16 ICL cache there beside the FP8 one)."""
        if self.context is not None:
            ck, cv, ik, iv = self.context
            named = {}
            for i in range(mf.COLUMN_BLOCKS):
                named[f"column.{i}.key"], named[f"column.{i}.value"] = ck[i], cv[i]
            for i in range(mf.ICL_BLOCKS):
                named[f"icl.{i}.key"], named[f"icl.{i}.value"] = ik[i], iv[i]
            flat = {k: np.ascontiguousarray(v).reshape(-1) for k, v in named.items()}
            return lambda name, start, count: flat[name][start:start + count]
        specs = self._specs()
        index = {name: i for i, (name, _, _) in enumerate(specs)}
        dtypes = {name: dtype for name, _, dtype in specs}
        buffers = {}

        def read(name, start, count):
            key = (count, dtypes[name])
            buf = buffers.get(key)
            if buf is None:
                buffers.clear()
                buf = buffers[key] = np.empty(count, dtypes[name])
            hip.check(hip.lib().irx_predictor_read_context(self.handle, index[name], start, count,
                                                           buf.ctypes.data_as(ctypes.c_void_p)))
            return buf

        return read

    def estimator_tensors(self, member: int):
        """One estimator's context tensors on the host, read out of HBM (or the
        host copy): (column keys [3][H+4,8,128,16], column values, ICL keys
        [12][8,N,64], ICL values), the slices of the context tensors
        (cpu.rs:4106-4123) at ``member``. The ICL tensors are FP16 for an
        optimize="auto" or "fast" context."""
        b, n, h = self.shape
        if not 0 <= member < b:
            raise ValueError(f"estimator {member} is outside 0..{b - 1}")
        read = self._tensor_source()
        col, icl = (h + 4) * 8 * 128 * 16, 8 * n * 64

        def take(name, size, shape):
            return np.array(read(name, member * size, size)).reshape(shape)

        ck = [take(f"column.{i}.key", col, (h + 4, 8, 128, 16)) for i in range(mf.COLUMN_BLOCKS)]
        cv = [take(f"column.{i}.value", col, (h + 4, 8, 128, 16)) for i in range(mf.COLUMN_BLOCKS)]
        ik = [take(f"icl.{i}.key", icl, (8, n, 64)) for i in range(mf.ICL_BLOCKS)]
        iv = [take(f"icl.{i}.value", icl, (8, n, 64)) for i in range(mf.ICL_BLOCKS)]
        return ck, cv, ik, iv

    def _persistable(self) -> cf.Metadata:
        if self.metadata is None:
            raise ValueError("this context has no identity metadata (built from bare tensors); "
                             "build it with Executor.build_context to save it")
        return self.metadata

    def _specs(self):
        icl_dtype = np.float32 if self.precision == hip.PRECISION_FP32 else np.float16
        return cf.context_tensor_specs(*self.shape, icl_dtype)

    def save_context(self, path) -> None:
        """Write the context as an IRCNTXT file, atomically, streaming its
        tensors from HBM when no host copy exists (FP16 ICL tensors, version
        2, for an optimize="auto" or "fast" context)."""
        meta = self._persistable()
        cf.write(path, meta, self._specs(), self._tensor_source())

    def context_encoded_len(self) -> int:
        return cf.encoded_len(self._persistable(), self._specs())

    def encode_context(self, sink) -> None:
        """Encode the context into the binary file-like `sink` as save_context writes it."""
        cf.encode(self._persistable(), self._specs(), self._tensor_source(), sink)

    def predict_raw(self, x: np.ndarray, progress=None) -> Prediction:
        """Every decoder output [B, Q, width] (Predictor::predict, predictor.rs:224-271)."""
        x = _f32(x)
        b, n, h = self.shape
        if x.ndim != 3 or x.shape[0] != b or x.shape[2] != h:
            raise ValueError(f"query shape {x.shape} does not match static context B={b} and H={h}")
        q = x.shape[1]
        logits = np.zeros((b, q, self.executor.width), np.float32)
        flags = np.zeros(q, np.uint8)
        if q:
            hip.check(hip.lib().irx_predictor_predict(
                self.handle, hip.fptr(x), q, hip.fptr(logits),
                flags.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), _progress(progress), None))
        cpu_rows = [int(r) for r in np.nonzero(flags)[0]]
        if cpu_rows:
            logits[:, cpu_rows, :] = np.nan
        return Prediction(logits, cpu_rows)

    def predict_logits(self, x: np.ndarray) -> Prediction:
        """[B, Q, C] logits, C = classes (or all 999 quantiles) (cpu.rs:2057-2108)."""
        p = self.predict_raw(x)
        return Prediction(np.ascontiguousarray(p.logits[:, :, : self.outputs()]), p.cpu_rows)

    def predict_probabilities(self, x: np.ndarray, temperature: float = 0.9, average_logits: bool = True):
        """Aggregated class probabilities [Q, C] (cpu.rs:2338-2348, 3873-3932)."""
        if not self.classes:
            raise ValueError("the context is a regression fit")
        p = self.predict_logits(x)
        if p.cpu_rows:
            # The reference re-runs these rows on its CPU path (cpu.rs:2072-2106);
            # this backend has none, so it refuses rather than return NaN.
            raise ValueError(f"rows {p.cpu_rows[:8]} hold the all-missing marker, which this backend does not "
                             "predict; use predict_logits and the CPU path for them")
        return aggregate_classifier_probabilities(p.logits, self.class_permutations, temperature, average_logits)

    def _check_bundle(self, query) -> None:
        meta = self.metadata
        if meta is None or query.model_sha256 != meta.model_sha256 or query.context_sha256 != meta.context_sha256:
            raise ValueError("query bundle model or context identity does not match the static context")

    def predict_bundle(self, query) -> Prediction:
        """Logits [B, Q, C] of an IRQUERY bundle made for exactly this context:
        its model and context identities must be this context's
        (StaticExecutor::predict_bundle, cpu.rs:2356-2373)."""
        self._check_bundle(query)
        return self.predict_logits(query.x)

    def predict_bundle_probabilities(self, query, temperature: float = 0.9, average_logits: bool = True):
        """Aggregated class probabilities [Q, C] of an IRQUERY bundle
        (StaticExecutor::predict_bundle_probabilities, cpu.rs:2373-2385)."""
        self._check_bundle(query)
        return self.predict_probabilities(query.x, temperature, average_logits)

    def predict_regression(self, x: np.ndarray, alphas=(0.05, 0.5, 0.95)):
        """(mean [Q], quantiles [Q, len(alphas)]) in standardized target units
        (predict_regression, cpu.rs:2305-2329)."""
        mean, quantiles = self.predict_regression_outputs(x, ("mean", "quantiles"), alphas)
        return mean, quantiles

    def predict_regression_outputs(self, x: np.ndarray, output_types=("mean",), alphas=()) -> list[np.ndarray]:
        """The requested regression outputs (RegressionOutput, quantiles.rs:26-63),
        in standardized target units: decoder outputs predicted into HBM and
        summarized there (quantiles::summarize on the GPU); only the summaries
        come back. Rows of the all-missing marker (cpu_rows) hold NaN."""
        if self.classes:
            raise ValueError("the context is a classification fit")
        for name in output_types:
            parse_regression_output(name, alphas)
        from . import hipmem

        x = _f32(x)
        b, n, h = self.shape
        if x.ndim != 3 or x.shape[0] != b or x.shape[2] != h:
            raise ValueError(f"query shape {x.shape} does not match static context B={b} and H={h}")
        q, width = x.shape[1], self.executor.width
        if q == 0:
            return [np.zeros((0,) + _regression_columns(t, alphas, width), np.float32) for t in output_types]
        dx = hipmem.DeviceArray.from_host(x)
        dl = hipmem.DeviceArray((b, q, width))
        flags = np.zeros(q, np.uint8)
        hip.check(hip.lib().irx_predictor_predict_device(self.handle, dx.ptr, q, dl.ptr,
                                                         flags.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))))
        outs = summarize_regression(self.executor.device, dl.ptr, (b, q, width), output_types, alphas)
        rows = np.nonzero(flags)[0]
        for o in outs:
            o[rows] = np.nan
        return outs


def aggregate_classifier_probabilities(logits: np.ndarray, perms: np.ndarray, temperature: float = 0.9,
                                       average_logits: bool = True) -> np.ndarray:
    """member[c] = logits[perm[e][c]]; mean over estimators; softmax(x / T);
    renormalize (aggregate_classifier_probabilities, cpu.rs:3873-3932)."""
    if not np.isfinite(temperature) or temperature <= 0:
        raise ValueError("softmax temperature must be positive and finite")
    b, q, c = logits.shape
    scale = np.float32(1.0) / np.float32(b)

    def softmax(v):
        z = v / np.float32(temperature)
        z = np.exp(z - z.max(axis=-1, keepdims=True))
        return z / z.sum(axis=-1, keepdims=True)

    total = np.zeros((q, c), np.float32)
    for e in range(b):
        member = logits[e][:, perms[e].astype(np.int64)]
        if not average_logits:
            member = softmax(member)
        total += member * scale
    if average_logits:
        total = softmax(total)
    return (total / total.sum(axis=-1, keepdims=True)).astype(np.float32)


REGRESSION_OUTPUTS = ("mean", "variance", "median", "quantiles", "raw_quantiles")


def parse_regression_output(name: str, alphas=()) -> str:
    """RegressionOutput::parse (quantiles.rs:43-63)."""
    if name not in REGRESSION_OUTPUTS:
        raise ValueError(f"unknown output_type {name!r}; expected mean, variance, median, quantiles, or raw_quantiles")
    if name == "quantiles" and not all(math.isfinite(float(a)) for a in alphas):
        raise ValueError("quantile levels must be finite")
    return name


def _regression_columns(name: str, alphas, width: int) -> tuple:
    return {"quantiles": (len(alphas),), "raw_quantiles": (width,)}.get(name, ())


def summarize_regression(device, decoded_ptr: int, shape, output_types, alphas=()) -> list[np.ndarray]:
    """quantiles::summarize (quantiles.rs:80-213) on the GPU over decoded
    quantiles [B, Q, K] already in HBM at `decoded_ptr`: one array per name in
    `output_types` ("mean" [Q], "variance" [Q], "median" [Q], "quantiles"
    [Q, len(alphas)], "raw_quantiles" [Q, K]), averaged over the B estimators."""
    from . import hipmem

    b, q, k = shape
    for name in output_types:
        parse_regression_output(name, alphas)
    levels = [float(a) for a in alphas] if "quantiles" in output_types else []
    if "median" in output_types:
        levels.append(0.5)
    levels = np.asarray(levels, np.float32)
    mean = hipmem.DeviceArray((q,))
    var = hipmem.DeviceArray((q,)) if "variance" in output_types else None
    at = hipmem.DeviceArray((q, len(levels))) if len(levels) else None
    raw = hipmem.DeviceArray((q, k)) if "raw_quantiles" in output_types else None
    hip.check(hip.lib().irx_regression_summary(
        device.handle, decoded_ptr, b, q, k, hip.fptr(levels) if len(levels) else None, len(levels), mean.ptr,
        var.ptr if var else None, at.ptr if at else None, raw.ptr if raw else None))
    at_host = at.to_host() if at else None
    n_alpha = len(alphas) if "quantiles" in output_types else 0
    got = {"mean": lambda: mean.to_host(), "variance": lambda: var.to_host(),
           "median": lambda: np.ascontiguousarray(at_host[:, -1]),
           "quantiles": lambda: np.ascontiguousarray(at_host[:, :n_alpha]),
           "raw_quantiles": lambda: raw.to_host()}
    return [got[name]() for name in output_types]
