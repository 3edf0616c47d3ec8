"""The `ironicl run` path over this backend (run_model, src/main.rs:197-223):
an IRMODEL artifact and either an IRINPUT bundle (uncached: build from its
training rows, predict the rest) or an IRQUERY bundle with the IRCNTXT context
it was made for (cached). Results print as the reference prints them
(print_logits / print_probabilities, main.rs:419-446) and can also be written
as IRLOGITS.

    python -m ironicl_amd.run --model M.irmodel --input Q.irquery --context C.irctx [--probabilities]
    python -m ironicl_amd.run --model M.irmodel --input I.irinput [--logits-out L.irlogits]
"""

from __future__ import annotations

import argparse
import sys

import numpy as np

from . import bundles, hip, tabicl


def format_logits(logits: np.ndarray) -> str:
    b, q, c = logits.shape
    lines = [f"shape: {b} {q} {c}"]
    for e in range(b):
        for r in range(q):
            lines.append(f"logits[{e},{r}]: " + " ".join(f"{v:.9e}" for v in logits[e, r]))
    return "\n".join(lines)


def format_probabilities(probabilities: np.ndarray) -> str:
    q, c = probabilities.shape
    lines = [f"shape: {q} {c}"]
    for r in range(q):
        lines.append(f"probabilities[{r}]: " + " ".join(f"{v:.9e}" for v in probabilities[r]))
    return "\n".join(lines)


def run(model, input_path, context=None, probabilities=False, logits_out=None, device=None) -> np.ndarray:
    """Runs one request; returns the logits [B, test rows, C] (or the
    probabilities [Q, C] with `probabilities`), written to `logits_out` as
    IRLOGITS when given."""
    executor = tabicl.Executor.from_model_file(model, device or hip.Device(0))
    if context is not None:
        query = bundles.StaticQueryBundle.read(input_path)
        static = executor.load_context(context)
        if probabilities:
            return static.predict_bundle_probabilities(query)
        logits = static.predict_bundle(query).logits
    else:
        if probabilities:
            raise ValueError("probabilities need a static context (--context)")
        logits = executor.predict_input_bundle(bundles.InputBundle.read(input_path)).logits
    if logits_out is not None:
        bundles.write_logits(logits_out, logits)
    return logits


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--model", required=True, help="IRMODEL v1 artifact")
    ap.add_argument("--input", required=True, help="IRQUERY (with --context) or IRINPUT bundle")
    ap.add_argument("--context", default=None, help="IRCNTXT static context the IRQUERY bundle was made for")
    ap.add_argument("--probabilities", action="store_true", help="aggregated class probabilities")
    ap.add_argument("--logits-out", default=None, help="also write the logits as IRLOGITS v1")
    args = ap.parse_args(argv)
    out = run(args.model, args.input, args.context, args.probabilities, args.logits_out)
    print(format_probabilities(out) if args.probabilities else format_logits(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
