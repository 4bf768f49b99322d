"""Shared test configuration: the ``gpu`` marker and numeric helpers."""

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X and the built libkx355.so")


@pytest.fixture(scope="session")
def device():
    """The GPU for ``gpu`` tests. The library must be built: a missing library fails, it does
    not skip."""
    import torch

    from kinomlx_amd import _lib

    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a visible GPU")
    _lib.load()
    return torch.device("cuda:0")


def cosine(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64))))


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-300))


# The north-star block bar: cosine >= 0.9995, and max abs error <= 2e-2 against the FP32
# evaluation. A bf16 output is compared elementwise beyond its own rounding:
# |got - ref| <= 2e-2 + half a bf16 ulp of ref. An FP32 output meets the literal 2e-2.
BLOCK_COS_MIN = 0.9995
BLOCK_ABS = 2e-2


def half_ulp_bf16(x) -> np.ndarray:
    """Half the bf16 spacing at |x| (the most one round-to-nearest to bf16 moves x): bf16 keeps
    8 significant bits, so the spacing in [2^e, 2^(e+1)) is 2^(e-7)."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return np.exp2(e - 8.0)


def half_ulp_fp16(x) -> np.ndarray:
    """Half the fp16 spacing at |x|: 2^(floor(log2 |x|) - 11) for normal values (11 significant
    bits), 2^-25 below the smallest normal 2^-14."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return np.exp2(e - 11.0)


def half_ulp(x, half: str = "bf16") -> np.ndarray:
    """Half the spacing of the output's 16-bit type (``"bf16"`` or ``"fp16"``) at |x|."""
    return half_ulp_fp16(x) if half == "fp16" else half_ulp_bf16(x)


def half_round_fp16(x) -> np.ndarray:
    """``x`` rounded to the nearest fp16 value (round half to even), as float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def half_round_bf16(x) -> np.ndarray:
    """``x`` rounded to the nearest bf16 value (round half to even), as float32."""
    import torch

    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def block_errors(got, ref, half: str = "bf16") -> dict:
    """Cosine, max abs error, and the max error beyond the output's own rounding to its 16-bit
    type ``half`` (with |ref| at that element)."""
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    diff = np.abs(g - r)
    excess = diff - half_ulp(r, half)
    i = int(np.argmax(excess))
    return {"cosine": cosine(g, r), "max_abs": float(diff.max()), "excess": float(excess.flat[i]),
            "ref_at_excess": float(np.abs(r.flat[i])), "max_ref": float(np.abs(r).max()),
            "rel_l2": rel_l2(g, r), "rms": float(np.sqrt(np.mean(diff * diff)))}


def assert_block_bar(got, ref, what: str = "", *, fp32_out: bool = False, context=None, half: str = "bf16") -> dict:
    """Assert the block bar and print the errors (``context``: the reference's own bf16-graph
    output on the same inputs, printed for comparison only; ``half``: the output's 16-bit type)."""
    assert np.all(np.isfinite(got)), what
    e = block_errors(got, ref, half)
    note = ""
    if context is not None:
        c = block_errors(context, ref, half)
        note = f" | reference {half} graph: max_abs {c['max_abs']:.4g} excess {c['excess']:.4g}"
    print(f"{what}: cosine {e['cosine']:.7f} rel_l2 {e['rel_l2']:.3g} max_abs {e['max_abs']:.4g} "
          f"excess {e['excess']:.4g} (|ref| {e['ref_at_excess']:.3g} there, max|ref| {e['max_ref']:.3g}){note}")
    assert e["cosine"] >= BLOCK_COS_MIN, (what, e)
    if fp32_out:
        assert e["max_abs"] <= BLOCK_ABS, (what, e)
    else:
        assert e["excess"] <= BLOCK_ABS, (what, e)
    return e


os.environ.setdefault("PYTHONHASHSEED", "0")


# At D = 4096 (benchmark configs 2-5) the synthetic N(0, 1) modulation gates amplify the bf16
# rounding of the GEMM operands (normalized input, attention output, FF hidden) to output errors of
# 0.05-0.15 for any bf16 execution, the reference's own included; which elements carry them depends
# on every rounding decision upstream, so no FP32 evaluation reproduces one bf16 execution there.
# Those blocks are held to the north-star cosine, to the relative-L2 bound the reference sets for
# its bf16 kernels (tests/models/ltx2/test_dense_attention.py:49-64: < 6e-3), to the noise a
# bf16 execution that stores bf16 exactly where this build does must carry (the RMS error against
# FP32 at most 1.25x that of the FP32 evaluation rounded at this build's bf16 points), and
# elementwise to the reference's own arithmetic: no element may miss the FP32 evaluation by more
# than the reference's bf16 graph (every array MLX materialises rounded to bf16,
# kinomlx/models/ltx2/transformer/transformer.py:16-45) misses it on the same inputs, beyond the
# output's own rounding. Each kernel stage at D = 4096 is held to the literal 2e-2 on its own in
# tests/test_block_stages_gpu.py.
BLOCK_REL_L2 = 6e-3
KX_NOISE_FACTOR = 1.25


def assert_block_parity(got, ref, what: str, *, ref_kx=None, graph=None, fp32_out: bool = False,
                        small: bool = True, half: str = "bf16") -> None:
    """Block parity against the FP32 evaluation ``ref``: the fixed block bar where bf16 storage
    admits it (``small``: D <= 1024); otherwise the cosine, ``BLOCK_REL_L2``, the storage-point
    noise bound against ``ref_kx`` (the FP32 evaluation rounded where this build stores bf16), and,
    with ``graph`` (the reference's own bf16 execution on the same inputs), the elementwise anchor:
    the largest error beyond the bf16 output rounding is at most the graph's (an FP32 ``got`` gets
    no rounding allowance: its max abs error is held to the graph's excess). ``half``: the 16-bit
    type (``"bf16"`` or ``"fp16"``) of the output, of ``ref_kx``'s storage points and of the graph."""
    if small:
        assert_block_bar(got, ref, what, fp32_out=fp32_out, context=graph, half=half)
        return
    e = block_errors(got, ref, half)
    note = ""
    c = None
    if graph is not None:
        c = block_errors(graph, ref, half)
        note = f" | reference {half} graph: rel_l2 {c['rel_l2']:.3g} max_abs {c['max_abs']:.4g} excess {c['excess']:.4g}"
    # the FP32 evaluation at this build's bf16 points, its output rounded as ``got`` is
    rounded = half_round_fp16(ref_kx) if half == "fp16" else half_round_bf16(ref_kx)
    k = block_errors(ref_kx if fp32_out else rounded, ref, half)
    print(f"{what}: cosine {e['cosine']:.7f} rel_l2 {e['rel_l2']:.3g} rms {e['rms']:.3g} (kx-point noise "
          f"{k['rms']:.3g}) max_abs {e['max_abs']:.4g} excess {e['excess']:.4g} (max|ref| {e['max_ref']:.3g}){note}")
    assert np.all(np.isfinite(got)), what
    assert e["cosine"] >= BLOCK_COS_MIN, (what, e)
    assert e["rel_l2"] <= BLOCK_REL_L2, (what, e)
    assert e["rms"] <= KX_NOISE_FACTOR * k["rms"], (what, e["rms"], k["rms"])
    if c is not None:
        mine = e["max_abs"] if fp32_out else e["excess"]
        assert mine <= c["excess"], (what, "elementwise error beyond the reference bf16 graph's", mine, c["excess"])
