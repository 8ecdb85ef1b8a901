"""Logit comparison shared by the GPU parity tests.

The model tolerance for logits (fp32 compute over fp16 weights and an fp16 KV cache, against the reference's fp32 CPU
forward): max |gpu - ref| <= 2e-2 absolute and max |gpu - ref| <= 1e-2 * max |ref|. Every comparison prints the
observed error next to the tolerance (visible with pytest -s / -rP), so the margin left is on record.
"""
import numpy as np

ATOL, RTOL = 2e-2, 1e-2


def logit_error(got, ref) -> tuple[float, float]:
    """(max abs error, max abs error / max |ref|)."""
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    err = float(np.max(np.abs(got - ref)))
    scale = float(np.max(np.abs(ref)))
    return err, err / scale if scale > 0 else float("inf") if err > 0 else 0.0


def assert_logits_close(got, ref, what=""):
    err, rel = logit_error(got, ref)
    print(f"[parity] {what}: max abs err {err:.3e} (tol {ATOL:g}), rel {rel:.3e} (tol {RTOL:g})", flush=True)
    assert err <= ATOL and rel <= RTOL, f"{what}: max abs err {err:.3e} (tol {ATOL:g}), rel {rel:.3e} (tol {RTOL:g})"
