"""The FP32 torch block reference used at full size is pinned against the numpy oracle. CPU."""

import numpy as np
import torch

import oracle
from kinomlx_amd import workloads
from tests import _torch_ref
from tests._blocks import ltx_case
from tests.conftest import max_abs


def test_torch_reference_matches_oracle_ltx_block():
    spec = workloads.LTXSpec(grid=(2, 3, 4), text_tokens=5, dim=256, heads=2, head_dim=128)
    p, op, inputs, pe = ltx_case(spec)
    x = inputs["x"][0].float().numpy()
    ctx = inputs["context"][0].float().numpy()
    ref = oracle.ltx_video_block(op, x, ctx, pe, heads=2)
    tp = {k: torch.from_numpy(np.asarray(v)) for k, v in op.items()}
    got = _torch_ref.ltx_video_block(tp, torch.from_numpy(x), torch.from_numpy(ctx),
                                     tuple(torch.from_numpy(t) for t in pe), heads=2).numpy()
    assert max_abs(got, ref) < 1e-4


def test_torch_reference_bf16_graph_matches_oracle_bf16_graph():
    """Both restatements of the reference's bf16 execution round at the same points: they agree
    up to rare one-ulp rounding flips, far below the bf16 graph's own error against FP32."""
    spec = workloads.LTXSpec(grid=(2, 3, 4), text_tokens=5, dim=256, heads=2, head_dim=128)
    p, op, inputs, pe = ltx_case(spec)
    x = inputs["x"][0].float().numpy()
    ctx = inputs["context"][0].float().numpy()
    fp32 = oracle.ltx_video_block(op, x, ctx, pe, heads=2)
    ref = oracle.ltx_video_block(op, x, ctx, pe, heads=2, bf16_graph=True)
    tp = {k: torch.from_numpy(np.asarray(v)) for k, v in op.items()}
    got = _torch_ref.ltx_video_block(tp, torch.from_numpy(x), torch.from_numpy(ctx),
                                     tuple(torch.from_numpy(t) for t in pe), heads=2, bf16_graph=True).numpy()
    assert np.mean(got == ref) > 0.95
    assert max_abs(got, ref) < 0.5 * max_abs(ref, fp32)


def test_bf16_graph_rounds_every_output_and_stays_close_to_fp32():
    """The bf16-graph mode returns bf16 values and differs from FP32 by rounding noise only
    (cosine > 0.9999); dropping a rounding point would leave non-bf16 values."""
    spec = workloads.LTXSpec(grid=(2, 3, 4), text_tokens=5, dim=256, heads=2, head_dim=128)
    _, op, inputs, pe = ltx_case(spec)
    x = inputs["x"][0].float().numpy()
    ctx = inputs["context"][0].float().numpy()
    fp32 = oracle.ltx_video_block(op, x, ctx, pe, heads=2)
    graph = oracle.ltx_video_block(op, x, ctx, pe, heads=2, bf16_graph=True)
    assert np.array_equal(graph, oracle.to_bf16(graph))
    assert not np.array_equal(fp32, oracle.to_bf16(fp32))
    cos = float(graph.ravel() @ fp32.ravel() / np.linalg.norm(graph) / np.linalg.norm(fp32))
    assert cos > 0.9999
    assert 0 < max_abs(graph, fp32) < 0.1


def _flux_small(ff):
    from tests._blocks import flux_case

    spec = workloads.FluxSpec(grid=(3, 4), text_tokens=5, dim=256, heads=2, head_dim=128, ff_hidden=384, ff=ff,
                              single=ff == "swiglu")
    return spec, flux_case(spec)


def test_torch_reference_matches_oracle_flux_double_and_config1_blocks():
    for ff in ("swiglu", "gelu"):
        spec, (p, op, _, inputs, rope) = _flux_small(ff)
        image, text = inputs["image"][0].float().numpy(), inputs["text"][0].float().numpy()
        rope_t = tuple(torch.from_numpy(t) for t in rope)
        tp = {k: torch.from_numpy(np.asarray(v)) for k, v in op.items()}
        for graph in (False, True):
            ri, rt = oracle.flux_double_block(op, image, text, op["image_mod"], op["text_mod"], rope,
                                              heads=spec.heads, ff=ff, bf16_graph=graph)
            gi, gt = _torch_ref.flux_double_block(tp, torch.from_numpy(image), torch.from_numpy(text),
                                                  tp["image_mod"], tp["text_mod"], rope_t, spec.heads, ff=ff,
                                                  bf16_graph=graph)
            if graph:  # rare one-ulp flips between the two restatements
                assert np.mean(gi.numpy() == ri) > 0.95 and np.mean(gt.numpy() == rt) > 0.95
            else:
                assert max_abs(gi.numpy(), ri) < 1e-4 and max_abs(gt.numpy(), rt) < 1e-4


def test_torch_reference_matches_oracle_flux_single_block():
    spec, (p, op, single, inputs, rope) = _flux_small("swiglu")
    x = np.concatenate([inputs["text"][0].float().numpy(), inputs["image"][0].float().numpy()])
    ref = oracle.flux_single_block(single, x, op["single_mod"], rope, heads=spec.heads, width=spec.dim)
    tp = {k: torch.from_numpy(np.asarray(v)) for k, v in single.items()}
    got = _torch_ref.flux_single_block(tp, torch.from_numpy(x), torch.from_numpy(op["single_mod"]),
                                       tuple(torch.from_numpy(t) for t in rope), spec.heads, spec.dim).numpy()
    assert max_abs(got, ref) < 1e-4


def test_kx_rounding_mode_matches_between_torch_and_oracle_and_sits_between_fp32_and_graph():
    """The ``kx`` mode (bf16 only where the MI355X path stores bf16) agrees between the two
    restatements; it rounds a strict subset of the graph's sites: its error against FP32 is
    nonzero and below the graph's, and the block output (an FP32 residual stream) is not rounded."""
    spec = workloads.LTXSpec(grid=(2, 3, 4), text_tokens=5, dim=256, heads=2, head_dim=128)
    _, op, inputs, pe = ltx_case(spec)
    x = inputs["x"][0].float().numpy()
    ctx = inputs["context"][0].float().numpy()
    fp32 = oracle.ltx_video_block(op, x, ctx, pe, heads=2)
    graph = oracle.ltx_video_block(op, x, ctx, pe, heads=2, bf16_graph=True)
    kx = oracle.ltx_video_block(op, x, ctx, pe, heads=2, rounding_mode="kx")
    tp = {k: torch.from_numpy(np.asarray(v)) for k, v in op.items()}
    got = _torch_ref.ltx_video_block(tp, torch.from_numpy(x), torch.from_numpy(ctx),
                                     tuple(torch.from_numpy(t) for t in pe), heads=2, rounding_mode="kx").numpy()
    assert max_abs(got, kx) < 0.25 * max_abs(kx, fp32)
    assert 0 < max_abs(kx, fp32) < max_abs(graph, fp32)
    assert not np.array_equal(kx, oracle.to_bf16(kx))
    assert oracle.KX_SITES == _torch_ref.KX_SITES


def test_kx_rounding_mode_flux_blocks():
    for ff in ("swiglu", "gelu"):
        spec, (p, op, single, inputs, rope) = _flux_small(ff)
        image, text = inputs["image"][0].float().numpy(), inputs["text"][0].float().numpy()
        rope_t = tuple(torch.from_numpy(t) for t in rope)
        tp = {k: torch.from_numpy(np.asarray(v)) for k, v in op.items()}
        outs = {}
        for mode in (None, "graph", "kx"):
            outs[mode] = oracle.flux_double_block(op, image, text, op["image_mod"], op["text_mod"], rope,
                                                  heads=spec.heads, ff=ff, rounding_mode=mode)
        gi, gt = _torch_ref.flux_double_block(tp, torch.from_numpy(image), torch.from_numpy(text), tp["image_mod"],
                                              tp["text_mod"], rope_t, spec.heads, ff=ff, rounding_mode="kx")
        for i, got in enumerate((gi.numpy(), gt.numpy())):
            err_kx = max_abs(outs["kx"][i], outs[None][i])
            assert max_abs(got, outs["kx"][i]) < 0.25 * err_kx
            assert 0 < err_kx < max_abs(outs["graph"][i], outs[None][i])
        if ff == "swiglu":
            x = np.concatenate([text, image])
            ref = {m: oracle.flux_single_block(single, x, op["single_mod"], rope, heads=spec.heads, width=spec.dim,
                                               rounding_mode=m) for m in (None, "graph", "kx")}
            sp = {k: torch.from_numpy(np.asarray(v)) for k, v in single.items()}
            got = _torch_ref.flux_single_block(sp, torch.from_numpy(x), torch.from_numpy(op["single_mod"]), rope_t,
                                               spec.heads, spec.dim, rounding_mode="kx").numpy()
            err_kx = max_abs(ref["kx"], ref[None])
            assert max_abs(got, ref["kx"]) < 0.25 * err_kx
            assert 0 < err_kx < max_abs(ref["graph"], ref[None])
