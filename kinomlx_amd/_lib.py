"""ctypes binding of ``libkx355.so`` (the C ABI declared in ``include/kx355.h``).

The library is loaded after ``torch`` so that its ``libamdhip64.so.7`` dependency resolves to the
HIP runtime torch already holds: device pointers and streams are then shared. There is no CPU or
PyTorch fallback anywhere behind these calls: a missing library raises.

Each ``launch_*`` function takes torch tensors, checks what the kernel assumes (device, dtype,
strides), and enqueues the kernel on the current torch stream.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "libkx355.so"

KX_OK = 0
KX_ERR_INVALID = -1
KX_ERR_UNSUPPORTED = -2
KX_ERR_LAUNCH = -3

KX_F32 = 0
KX_BF16 = 1
KX_F16 = 2
KX_NORM_RMS = 0
KX_NORM_LAYER = 1
KX_NORM_IN_F32 = 1 << 4
KX_FP4_MX = 0
KX_FP4_NV = 1
KX_ROPE_NONE = 0
KX_ROPE_SPLIT = 1
KX_ROPE_PAIR = 2
EPI_BIAS = 1
EPI_ACT_GELU_TANH = 1 << 4
EPI_ACT_SILU = 2 << 4
EPI_ACT_SIGMOID2 = 3 << 4
EPI_ACT_SIGMOID = 4 << 4
EPI_GATED_RESIDUAL = 1 << 8
EPI_RESID_F32 = 1 << 9
EPI_OUT_F32 = 1 << 10

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# Entry point -> argument types (every function returns int).
SIGNATURES: dict[str, list] = {
    "kx_adaln_norm_bf16": [_P, _I64, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _F, _I, _P],
    "kx_rmsnorm_rope_bf16": [
        _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I, _F, _F, _I, _P, _P, _I64, _I64, _I64, _I,
        _I64, _P,
    ],
    "kx_qk_rmsnorm_rope_bf16": [
        _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _I, _F, _F, _P, _P, _I64, _I64, _I64, _I,
        _P,
    ],
    "kx_rope_split_bf16": [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _I, _P],
    "kx_rope_pair_bf16": [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _I, _P],
    "kx_attention_fwd_bf16": [
        _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _I64, _P,
    ],
    "kx_attention_gqa_fwd_bf16": [
        _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _I64, _P,
    ],
    "kx_attention_bias_fwd_bf16": [
        _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _I64, _P, _I64, _I64,
        _I64, _P,
    ],
    "kx_attention_split_fwd_bf16": [
        _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _I64, _P, _I64, _I64,
        _I64, _P, _I64, _I, _P,
    ],
    "kx_gemm_bf16": [
        _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _I64, _P, _I64, _I64, _P,
    ],
    "kx_gemm_splitk_bf16": [
        _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _I64, _P, _I64, _I64, _P, _I64, _I, _P,
    ],
    "kx_gemm_splitk_noalloc_bf16": [
        _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _I64, _P, _I64, _I64, _I, _P,
    ],
    "kx_qgemm_affine_bf16": [
        _P, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _I, _P, _I64, _P, _I64,
        _I64, _P,
    ],
    "kx_dequant_affine_bf16": [_P, _P, _P, _P, _I64, _I64, _I, _I, _P],
    "kx_quantize_affine_bf16": [_P, _I64, _P, _P, _P, _I64, _I64, _I, _I, _P],
    "kx_qweight_tile_affine": [_P, _P, _P, _P, _P, _I64, _I64, _I, _I, _P],
    "kx_qgemm_affine_tiled_bf16": [
        _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _P, _I64, _P, _I64, _I64, _P,
    ],
    "kx_table_add_f32": [_P, _I, _P, _I, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I, _P],
    "kx_gemm_qknorm_rope_bf16": [
        _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _I, _F, _F, _P, _P, _I64, _I64,
        _I64, _I64, _P,
    ],
    "kx_qgemm_mxfp8_bf16": [
        _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _P, _I64, _P, _I64, _I64, _P,
    ],
    "kx_dequant_mxfp8_bf16": [_P, _P, _P, _I64, _I64, _I, _I, _P],
    "kx_dequant_fp4_bf16": [_P, _P, _P, _I64, _I64, _I, _I, _P],
    "kx_quantize_fp4_bf16": [_P, _I64, _P, _P, _I64, _I64, _I, _I, _P],
    "kx_quantize_mxfp8_bf16": [_P, _I64, _P, _P, _I64, _I64, _I, _P],
    "kx_gelu_tanh_bf16": [_P, _P, _I64, _P],
    "kx_silu_bf16": [_P, _P, _I64, _P],
    "kx_swiglu_bf16": [_P, _I64, _P, _I64, _I64, _I64, _P],
    "kx_modulate_bf16": [_P, _I64, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _P],
    "kx_gated_residual_bf16": [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _P],
    "kx_timestep_embedding": [_P, _P, _I64, _I64, _I, _F, _F, _P],
    "kx_ltx_rope_tables": [_P, _I64, _I, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P],
    "kx_euler_velocity_step": [_P, _P, _P, _I64, _I, _F, _P],
    "kx_euler_step": [_P, _I, _P, _I, _P, _I64, _F, _P],
    "kx_to_denoised": [_P, _I, _P, _I, _P, _P, _I64, _I64, _I64, _P],
    "kx_mask_composite": [_P, _I, _P, _I, _P, _P, _I64, _I64, _P],
    "kx_all_finite": [_P, _I64, _I, _P, _P],
}

# fp16 entry points: the bf16 namesake's arguments with fp16 16-bit tensors (include/kx355.h)
F16_ENTRIES = (
    "kx_adaln_norm", "kx_rmsnorm_rope", "kx_qk_rmsnorm_rope", "kx_rope_split", "kx_rope_pair",
    "kx_attention_fwd", "kx_attention_gqa_fwd", "kx_attention_bias_fwd", "kx_attention_split_fwd", "kx_gemm",
    "kx_gemm_splitk", "kx_gelu_tanh", "kx_silu", "kx_swiglu", "kx_modulate", "kx_gated_residual",
)
for _base in F16_ENTRIES:
    SIGNATURES[f"{_base}_f16"] = SIGNATURES[f"{_base}_bf16"]
del _base

_lib: ctypes.CDLL | None = None


class KernelError(RuntimeError):
    """A kx355 entry point returned an error code."""


def load() -> ctypes.CDLL:
    """Load ``libkx355.so`` once; raise if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY_PATH.exists():
        raise RuntimeError(
            f"the kx355 HIP library is not built ({LIBRARY_PATH} missing); "
            "run `python -m kinomlx_amd.csrc.build`"
        )
    lib = ctypes.CDLL(os.fspath(LIBRARY_PATH), mode=ctypes.RTLD_LOCAL)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    lib.kx_abi_version.restype = ctypes.c_int
    lib.kx_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib


def available() -> bool:
    """Whether the library is built and a GPU is visible to torch."""
    return LIBRARY_PATH.exists() and torch.cuda.is_available()


class LaunchTimer:
    """Optional per-launch timing: while installed, each entry point call is bracketed by two
    ``torch.cuda.Event`` records on the current stream (the stream the kernel runs on)."""

    def __init__(self) -> None:
        self.records: list[tuple[str, tuple, torch.cuda.Event, torch.cuda.Event]] = []

    def durations_ms(self) -> list[tuple[str, tuple, float]]:
        """(entry point, its C arguments, milliseconds) per recorded launch."""
        torch.cuda.synchronize()
        return [(name, args, start.elapsed_time(end)) for name, args, start, end in self.records]


_timer: LaunchTimer | None = None


def set_timer(timer: LaunchTimer | None) -> None:
    """Install (or remove with None) a ``LaunchTimer``."""
    global _timer
    _timer = timer


def _call(name: str, *args, unsupported_ok: bool = False) -> int:
    """Run one entry point (timed when a LaunchTimer is set); raise on an error code, except
    KX_ERR_UNSUPPORTED when ``unsupported_ok`` (then the code is returned and nothing ran)."""
    lib = load()
    timer = _timer
    if timer is not None:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
    rc = getattr(lib, name)(*args)
    if timer is not None:
        end.record()
        timer.records.append((name, args, start, end))
    if rc == KX_ERR_UNSUPPORTED and unsupported_ok:
        if timer is not None:
            timer.records.pop()
        return rc
    if rc != KX_OK:
        message = lib.kx_last_error().decode(errors="replace")
        raise KernelError(f"{name} failed ({rc}): {message}")
    return rc


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _check_gpu(name: str, *tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError(f"{name}: the MI355X kernels take GPU tensors, got one on {t.device}")


HALF_DTYPES = (torch.bfloat16, torch.float16)


def _suffix(t: torch.Tensor, name: str) -> str:
    """The entry-point suffix for a 16-bit activation tensor: ``bf16`` or ``f16``."""
    if t.dtype == torch.bfloat16:
        return "bf16"
    if t.dtype == torch.float16:
        return "f16"
    raise ValueError(f"{name}: needs float16 or bfloat16 activations, got {t.dtype}")


def _same_dtype(name: str, dtype: torch.dtype, *tensors) -> None:
    for t in tensors:
        if t is not None and t.dtype != dtype:
            raise ValueError(f"{name}: every 16-bit tensor must be {dtype}, got {t.dtype}")


def _weight_code(w: torch.Tensor, name: str) -> int:
    codes = {torch.float32: KX_F32, torch.bfloat16: KX_BF16, torch.float16: KX_F16}
    if w.dtype not in codes:
        raise ValueError(f"{name}: norm weight must be float32, bfloat16 or float16, got {w.dtype}")
    return codes[w.dtype]


def _rows(t: torch.Tensor, name: str) -> tuple[int, int, int]:
    """(rows, width, row stride) of a tensor whose last axis is contiguous and whose leading
    axes flatten into rows of one stride."""
    if t.dim() < 1:
        raise ValueError(f"{name}: needs at least one axis")
    width = t.shape[-1]
    if t.stride(-1) != 1 and width > 1:
        raise ValueError(f"{name}: last axis must be contiguous")
    if t.dim() == 1:
        return 1, width, width
    rows = t.numel() // width if width else 0
    stride = t.stride(-2)
    # leading axes must collapse into one stride
    expected = stride
    for axis in range(t.dim() - 2, -1, -1):
        if t.shape[axis] != 1 and t.stride(axis) != expected:
            raise ValueError(f"{name}: leading axes do not flatten into evenly strided rows")
        expected *= t.shape[axis]
    return rows, width, max(stride, width)


def _mod_rows(vec: torch.Tensor, rows: int, width: int, name: str) -> tuple[int, int]:
    """(mod_div, mod_stride) for an fp32 modulation tensor broadcast over ``rows`` rows: one
    row ``(width,)``/``(1, .., width)``, one per batch ``(B, 1, width)``, or one per row."""
    if vec.dtype != torch.float32 or vec.shape[-1] != width or vec.stride(-1) != 1:
        raise ValueError(f"{name}: modulation must be fp32 with a contiguous last axis {width}")
    count = vec.numel() // width
    if count == 1:
        return 1, 0
    if rows % count:
        raise ValueError(f"{name}: {count} modulation rows do not divide {rows} rows")
    stride = vec.stride(-2) if vec.dim() >= 2 and vec.shape[-2] != 1 else vec.stride(0)
    return rows // count, stride


# ---- launches -----------------------------------------------------------------------------------


def _shared_mod_rows(shift, scale, rows: int, width: int, name: str) -> tuple[int, int]:
    """The one (mod_div, mod_stride) layout that ``shift`` and ``scale`` must share: the
    kernels index both with it."""
    layout = _mod_rows(shift, rows, width, f"{name} shift")
    if _mod_rows(scale, rows, width, f"{name} scale") != layout:
        raise ValueError(f"{name}: shift and scale must share one layout")
    return layout


def launch_adaln_norm(x, out, shift, scale, eps: float, kind: int) -> None:
    """``out`` is bf16 or fp16; ``x`` is of the same type or fp32 (a residual stream carried in
    fp32)."""
    _check_gpu("adaln_norm", x, out, shift, scale)
    suffix = _suffix(out, "adaln_norm out")
    if x.dtype == torch.float32:
        kind |= KX_NORM_IN_F32
    elif x.dtype != out.dtype:
        raise ValueError(f"adaln_norm: x must be {out.dtype} or float32, got {x.dtype}")
    rows, dim, ldx = _rows(x, "adaln_norm x")
    _, _, ldy = _rows(out, "adaln_norm out")
    div, stride = (1, 0)
    if shift is not None:
        div, stride = _shared_mod_rows(shift, scale, rows, dim, "adaln_norm")
    _call(
        f"kx_adaln_norm_{suffix}", _ptr(x), ldx, _ptr(out), ldy, rows, dim, _ptr(shift), _ptr(scale),
        div, stride, eps, kind, _stream(),
    )


def launch_rmsnorm_rope(
    x, out, weight, eps: float, weight_offset: float, *, norm_width: int, rope_kind: int = 0,
    cos=None, sin=None, table_ld: int = 0, table_hs: int = 0, tokens: int = 0,
    table_batched: bool = False, head_dim: int = 0,
) -> None:
    _check_gpu("rmsnorm_rope", x, out, weight, cos, sin)
    suffix = _suffix(x, "rms_norm")
    _same_dtype("rms_norm", x.dtype, out)
    rows, dim, ldx = _rows(x, "rmsnorm x")
    _, _, ldy = _rows(out, "rmsnorm out")
    w_dtype = _weight_code(weight, "rms_norm")
    if not weight.is_contiguous():
        raise ValueError("rms_norm weight must be contiguous")
    _call(
        f"kx_rmsnorm_rope_{suffix}", _ptr(x), ldx, _ptr(out), ldy, rows, dim, norm_width, _ptr(weight),
        w_dtype, eps, weight_offset, rope_kind, _ptr(cos), _ptr(sin), table_ld, table_hs, tokens,
        int(table_batched), head_dim, _stream(),
    )


def launch_qk_rmsnorm_rope(xq, xk, yq, yk, wq, wk, eps: float, *, cos, sin, table_ld: int, table_hs: int,
                           tokens: int, table_batched: bool) -> bool:
    """One pass for the Q and K rows of the same tokens; False (nothing launched) when the shape
    or alignment is outside the fused kernel's contract."""
    _check_gpu("qk_rmsnorm_rope", xq, xk, yq, yk, wq, wk, cos, sin)
    rows, dim, ldq = _rows(xq, "qk_rmsnorm_rope q")
    rows_k, dim_k, ldk = _rows(xk, "qk_rmsnorm_rope k")
    _, _, ldyq = _rows(yq, "qk_rmsnorm_rope q out")
    _, _, ldyk = _rows(yk, "qk_rmsnorm_rope k out")
    if (rows_k, dim_k) != (rows, dim) or wq.dtype != wk.dtype:
        raise ValueError("qk_rmsnorm_rope: q and k must have one shape and one weight dtype")
    suffix = _suffix(xq, "qk_rmsnorm_rope")
    _same_dtype("qk_rmsnorm_rope", xq.dtype, xk, yq, yk)
    w_dtype = _weight_code(wq, "rms_norm")
    code = _call(
        f"kx_qk_rmsnorm_rope_{suffix}", _ptr(xq), ldq, _ptr(xk), ldk, _ptr(yq), ldyq, _ptr(yk), ldyk, rows, dim,
        _ptr(wq), _ptr(wk), w_dtype, eps, 0.0, _ptr(cos), _ptr(sin), table_ld, table_hs, tokens,
        int(table_batched), _stream(), unsupported_ok=True,
    )
    return code == KX_OK


def launch_rope_split(x, out, cos_tm, sin_tm, *, batch, tokens, heads, half, table_batched) -> None:
    _check_gpu("rope_split", x, out, cos_tm, sin_tm)
    suffix = _suffix(x, "rope")
    _same_dtype("rope", x.dtype, out)
    _, _, ldx = _rows(x, "rope x")
    _, _, ldy = _rows(out, "rope out")
    _call(
        f"kx_rope_split_{suffix}", _ptr(x), ldx, _ptr(out), ldy, batch, tokens, heads, half,
        _ptr(cos_tm), _ptr(sin_tm), int(table_batched), _stream(),
    )


def launch_rope_pair(x, out, cos, sin, *, heads, head_dim, table_ld, table_hs, tokens, table_batched) -> None:
    _check_gpu("rope_pair", x, out, cos, sin)
    suffix = _suffix(x, "rope")
    _same_dtype("rope", x.dtype, out)
    rows, _, ldx = _rows(x, "rope x")
    _, _, ldy = _rows(out, "rope out")
    _call(
        f"kx_rope_pair_{suffix}", _ptr(x), ldx, _ptr(out), ldy, rows, heads, head_dim, _ptr(cos),
        _ptr(sin), table_ld, table_hs, tokens, int(table_batched), _stream(),
    )


def launch_attention(q, k, v, out, *, batch, tq, tk, heads, head_dim, scale, gate=None, kv_heads=None,
                     bias=None, bias_strides=None) -> None:
    _check_gpu("attention", q, k, v, out, gate, bias)
    sfx = _suffix(q, "attention")
    _same_dtype("attention", q.dtype, k, v, out, gate)
    ld_gate = 0
    if gate is not None:
        _, _, ld_gate = _rows(gate, "attention gate")
    if bias is not None and (bias.dtype != q.dtype or bias_strides is None):
        raise ValueError(f"attention bias: {q.dtype} values with (batch, head, query) strides")
    splits = attention_splits(batch, tq, tk, heads)
    if splits > 1:
        chunk = -(-(-(-tk // splits)) // 64) * 64
        used = -(-tk // chunk)
        work = torch.empty(used * batch * heads * tq * (head_dim + 2), dtype=torch.float32, device=q.device)
        _call(
            f"kx_attention_split_fwd_{sfx}", _ptr(q), q.stride(-2), _ptr(k), k.stride(-2), _ptr(v), v.stride(-2),
            _ptr(out), out.stride(-2), batch, tq, tk, heads, kv_heads or heads, head_dim, scale, _ptr(gate), ld_gate,
            _ptr(bias), *(bias_strides or (0, 0, 0)), _ptr(work), work.numel() * 4, splits, _stream(),
        )
        return
    if bias is not None:
        _call(
            f"kx_attention_bias_fwd_{sfx}", _ptr(q), q.stride(-2), _ptr(k), k.stride(-2), _ptr(v), v.stride(-2),
            _ptr(out), out.stride(-2), batch, tq, tk, heads, kv_heads or heads, head_dim, scale, _ptr(gate), ld_gate,
            _ptr(bias), *bias_strides, _stream(),
        )
        return
    if kv_heads is not None and kv_heads != heads:
        _call(
            f"kx_attention_gqa_fwd_{sfx}", _ptr(q), q.stride(-2), _ptr(k), k.stride(-2), _ptr(v),
            v.stride(-2), _ptr(out), out.stride(-2), batch, tq, tk, heads, kv_heads, head_dim, scale,
            _ptr(gate), ld_gate, _stream(),
        )
        return
    _call(
        f"kx_attention_fwd_{sfx}", _ptr(q), q.stride(-2), _ptr(k), k.stride(-2), _ptr(v),
        v.stride(-2), _ptr(out), out.stride(-2), batch, tq, tk, heads, head_dim, scale,
        _ptr(gate), ld_gate, _stream(),
    )


def attention_splits(batch: int, tq: int, tk: int, heads: int) -> int:
    """Key slices for an attention call whose query tiles (384 queries x 1 head) fill under half
    the 256 CUs and that has at least 1024 keys: about 512 workgroups, at least 256 keys per
    slice, at most 16 slices; 1 means no split."""
    blocks = -(-tq // 384) * heads * batch
    if blocks >= 128 or tk < 1024:
        return 1
    return max(1, min(16, -(-512 // blocks), tk // 256))


def _dtype_flags(out, resid, name: str, half: torch.dtype = torch.bfloat16) -> int:
    """Epilogue flags for an fp32 output and an fp32 residual (``half``, the operands' 16-bit
    type, otherwise)."""
    flags = 0
    if out.dtype == torch.float32:
        flags |= EPI_OUT_F32
    elif out.dtype != half:
        raise ValueError(f"{name}: the output must be {half} or float32, got {out.dtype}")
    if resid is not None:
        if resid.dtype == torch.float32:
            flags |= EPI_RESID_F32
        elif resid.dtype != half:
            raise ValueError(f"{name}: the residual must be {half} or float32, got {resid.dtype}")
    return flags


def launch_gemm(a, w, out, *, bias=None, flags: int = 0, resid=None, gate=None) -> None:
    _check_gpu("gemm", a, w, out, bias, resid, gate)
    sfx = _suffix(a, "linear")
    _same_dtype("linear", a.dtype, w, bias)
    flags |= _dtype_flags(out, resid, "linear", a.dtype)
    m, k, lda = _rows(a, "linear input")
    n, kw, ldw = _rows(w, "linear weight")
    if kw != k:
        raise ValueError(f"linear: input width {k} does not match weight width {kw}")
    _, _, ldc = _rows(out, "linear output")
    ldr, div, stride = 0, 1, 0
    if resid is not None:
        _, _, ldr = _rows(resid, "linear residual")
        div, stride = _mod_rows(gate, m, n, "linear gate")
    plan = tail_split(m, n, k)
    # a gate that changes with the row block (stride != 0) keeps the plain tiling: the tail call
    # would index its rows from zero
    if plan is not None and (gate is None or stride == 0) and a.data_ptr() % 16 == 0 \
            and w.data_ptr() % 16 == 0 and lda <= (1 << 22) and ldw <= (1 << 22):
        # whole rounds of 256x256 tiles over the first rows, the tail rows as K slices filling one
        # round. The tail goes first: its rows are the input's last, the ones its producer wrote
        # most recently (the likeliest to be in the memory-side cache), and its pass leaves the
        # weight in that cache for the head (the down projection's head 923 -> 907 us).
        rows, tail_splits = plan
        tail = m - rows
        work = torch.empty(tail_splits * tail * n, dtype=torch.float32, device=a.device)
        # row ``rows`` of each operand from its flattened row stride (the leading axes of an N-D
        # tensor are not rows)
        a_tail = a.data_ptr() + rows * lda * a.element_size()
        out_tail = out.data_ptr() + rows * ldc * out.element_size()
        resid_tail = None if resid is None else resid.data_ptr() + rows * ldr * resid.element_size()
        _call(
            f"kx_gemm_splitk_{sfx}", a_tail, lda, _ptr(w), ldw, _ptr(bias), out_tail, ldc, tail, n, k,
            flags, resid_tail, ldr, _ptr(gate), div, stride, _ptr(work), work.numel() * 4, tail_splits, _stream(),
        )
        _call(
            f"kx_gemm_{sfx}", _ptr(a), lda, _ptr(w), ldw, _ptr(bias), _ptr(out), ldc, rows, n, k, flags,
            _ptr(resid), ldr, _ptr(gate), div, stride, _stream(),
        )
        return
    splits = splitk_splits(m, n, k)
    if splits > 1 and a.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0 and lda <= (1 << 22) and ldw <= (1 << 22):
        work = torch.empty(splits * m * n, dtype=torch.float32, device=a.device)
        _call(
            f"kx_gemm_splitk_{sfx}", _ptr(a), lda, _ptr(w), ldw, _ptr(bias), _ptr(out), ldc, m, n, k, flags,
            _ptr(resid), ldr, _ptr(gate), div, stride, _ptr(work), work.numel() * 4, splits, _stream(),
        )
        return
    _call(
        f"kx_gemm_{sfx}", _ptr(a), lda, _ptr(w), ldw, _ptr(bias), _ptr(out), ldc, m, n, k, flags,
        _ptr(resid), ldr, _ptr(gate), div, stride, _stream(),
    )


def launch_gemm_qknorm_rope(a, w, out, *, bias, q_end: int, k_end: int, norm_q, norm_k, eps: float,
                            weight_offset: float, cos, sin, table_ld: int, table_hs: int, table_rows: int,
                            table_bs: int) -> None:
    """``out = a @ w.T + bias`` with per-head (128) RMSNorm + adjacent-pair RoPE applied to the
    query columns ``[0, q_end)`` and key columns ``[q_end, k_end)`` in the GEMM epilogue."""
    _check_gpu("gemm_qknorm_rope", a, w, out, bias, norm_q, norm_k, cos, sin)
    m, k, lda = _rows(a, "qk-norm projection input")
    n, kw, ldw = _rows(w, "qk-norm projection weight")
    if kw != k:
        raise ValueError(f"qk-norm projection: input width {k} does not match weight width {kw}")
    _, nout, ldc = _rows(out, "qk-norm projection output")
    if nout != n or out.dtype != torch.bfloat16:
        raise ValueError("qk-norm projection: out must be bf16 rows of the weight's output width")
    if norm_q.dtype != norm_k.dtype or norm_q.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("qk-norm projection: norm weights must both be fp32 or both bf16")
    if norm_q.shape != (128,) or norm_k.shape != (128,) or not (norm_q.is_contiguous() and norm_k.is_contiguous()):
        raise ValueError("qk-norm projection: norm weights must be contiguous (128,)")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise ValueError("qk-norm projection: rotary tables must be fp32")
    _call(
        "kx_gemm_qknorm_rope_bf16", _ptr(a), lda, _ptr(w), ldw, _ptr(bias), _ptr(out), ldc, m, n, k, q_end, k_end,
        _ptr(norm_q), _ptr(norm_k), KX_BF16 if norm_q.dtype == torch.bfloat16 else KX_F32, float(eps),
        float(weight_offset), _ptr(cos), _ptr(sin), table_ld, table_hs, table_rows, table_bs, _stream(),
    )


def tail_split(m: int, n: int, k: int) -> tuple[int, int] | None:
    """``(rows, splits)`` when a product's 256x256 tiles would end in a partial round of
    workgroups (e.g. 9216 x 4096: 576 tiles, 2.25 rounds on 256 CUs): the first ``rows`` rows run as
    whole rounds of 256x256 tiles, and the remaining rows as ``splits`` K slices of 256x256 tiles,
    which take one round (or, for a tail over half a round, a few rounds) of a fraction of a
    tile's work each; the slices' fp32 partial products are summed by the split-K reduction, which
    applies the epilogue. None when the product takes the plain tiling."""
    # the slices of the tail are a quarter of a tile's K or less: worth their partial products and
    # reduction only for long K (the 9216 x 4096 x 16384 down projection: 1.33 -> 1.16 ms; at
    # K = 4096 the tail costs more than the partial round it replaces)
    if m < 2048 or n % 256 or n < 1024 or k < 8192:
        return None
    tiles_n = n // 256
    rounds = (m // 256) * tiles_n // 256
    if rounds < 1 or (rounds * 256) % tiles_n:
        return None
    rows = rounds * 256 // tiles_n * 256
    tail_tiles = -(-(m - rows) // 256) * tiles_n
    if tail_tiles == 0 or tail_tiles > 256:
        return None
    splits = 1
    if tail_tiles <= 128:
        # the most slices that still fit one round
        for cand in (2, 4, 8):
            if tail_tiles * cand <= 256 and k % (64 * cand) == 0 and k // cand >= 512:
                splits = cand
    else:
        # a tail over half a round (27 280 rows: 176 tiles): the slice count with the fewest
        # rounds of 1/splits tiles, under the one full round the tail takes unsplit
        best = 1.0
        for cand in (2, 4, 8):
            cost = -(-tail_tiles * cand // 256) / cand
            if cost < best - 1e-9 and k % (64 * cand) == 0 and k // cand >= 512:
                splits, best = cand, cost
    return (rows, splits) if splits > 1 else None


def splitk_splits(m: int, n: int, k: int) -> int:
    """K slices for a product whose output tiles (64 x 128) leave most of the 256 CUs idle:
    the most slices (up to 16) that keep at most 512 workgroups, a slice of at least 256 and a
    whole number of 64-wide stages per slice; 1 means no split."""
    if m > 512 or n <= 64 or n % 4 or k < 1024:
        return 1
    tiles = -(-m // 64) * -(-n // 128)
    if tiles >= 128:
        return 1
    best = 1
    for splits in (2, 4, 8, 16):
        if tiles * splits <= 512 and k % (64 * splits) == 0 and k // splits >= 256:
            best = splits
    return best


def launch_qgemm(a, words, scales, biases, out, *, n, k, group_size, bits, bias=None,
                 flags: int = 0, resid=None, gate=None) -> None:
    _check_gpu("qgemm", a, words, scales, biases, out, bias, resid, gate)
    flags |= _dtype_flags(out, resid, "quantized linear")
    m, ka, lda = _rows(a, "quantized linear input")
    if ka != k:
        raise ValueError(f"quantized linear: input width {ka} does not match {k}")
    _, _, ldc = _rows(out, "quantized linear output")
    ldr, div, stride = 0, 1, 0
    if resid is not None:
        _, _, ldr = _rows(resid, "quantized linear residual")
        div, stride = _mod_rows(gate, m, n, "quantized linear gate")
    _call(
        "kx_qgemm_affine_bf16", _ptr(a), lda, _ptr(words), _ptr(scales), _ptr(biases), _ptr(bias),
        _ptr(out), ldc, m, n, k, group_size, bits, flags, _ptr(resid), ldr, _ptr(gate), div,
        stride, _stream(),
    )


def launch_qgemm_mxfp8(a, words, scales, out, *, n, k, group_size=32, bias=None, flags: int = 0, resid=None,
                       gate=None) -> None:
    """``out = epilogue(a @ dequant(words, scales).T)`` for mxfp8 weights (words (n, k / 4) uint32,
    scales (n, k / 32) uint8)."""
    _check_gpu("qgemm_mxfp8", a, words, scales, out, bias, resid, gate)
    if words.shape != (n, k // 4) or scales.shape != (n, k // group_size) or scales.dtype != torch.uint8:
        raise ValueError("mxfp8 linear: words must be (n, k / 4) and scales (n, k / 32) uint8")
    flags |= _dtype_flags(out, resid, "quantized linear")
    m, ka, lda = _rows(a, "quantized linear input")
    if ka != k:
        raise ValueError(f"quantized linear: input width {ka} does not match {k}")
    _, _, ldc = _rows(out, "quantized linear output")
    ldr, div, stride = 0, 1, 0
    if resid is not None:
        _, _, ldr = _rows(resid, "quantized linear residual")
        div, stride = _mod_rows(gate, m, n, "quantized linear gate")
    _call(
        "kx_qgemm_mxfp8_bf16", _ptr(a), lda, _ptr(words), _ptr(scales), _ptr(bias), _ptr(out), ldc, m, n, k,
        group_size, flags, _ptr(resid), ldr, _ptr(gate), div, stride, _stream(),
    )


def launch_dequant_mxfp8(words, scales, out, *, n, k, group_size=32, transposed: bool = False) -> None:
    """The bf16 (n, k) weight of mxfp8 ``words``/``scales``: the (n, k / 4) layout, or with
    ``transposed`` the (k, n / 4) layout quantized from ``weight.T``."""
    _check_gpu("dequant_mxfp8", words, scales, out)
    rows, cols = (k, n) if transposed else (n, k)
    if words.shape != (rows, cols // 4) or scales.shape != (rows, cols // group_size):
        raise ValueError("dequant_mxfp8: packed shapes do not match (n, k)")
    if out.shape != (n, k) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("dequant_mxfp8: out must be a contiguous bf16 (n, k) tensor")
    _call("kx_dequant_mxfp8_bf16", _ptr(words), _ptr(scales), _ptr(out), n, k, group_size, int(transposed),
          _stream())


def launch_dequant_fp4(words, scales, out, *, n, k, group_size, scale_kind) -> None:
    """The bf16 (n, k) weight of FP4 ``words`` (n, k / 8) / ``scales`` (n, k / group_size) uint8."""
    _check_gpu("dequant_fp4", words, scales, out)
    if words.shape != (n, k // 8) or scales.shape != (n, k // group_size) or scales.dtype != torch.uint8:
        raise ValueError("dequant_fp4: words must be (n, k / 8) and scales (n, k / group_size) uint8")
    if out.shape != (n, k) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("dequant_fp4: out must be a contiguous bf16 (n, k) tensor")
    _call("kx_dequant_fp4_bf16", _ptr(words.contiguous()), _ptr(scales.contiguous()), _ptr(out), n, k, group_size,
          scale_kind, _stream())


def launch_quantize_fp4(w, words, scales, *, group_size: int, scale_kind: int) -> None:
    """FP4 (words, scales) <- bf16 weight w (n, k) with contiguous rows."""
    _check_gpu("quantize_fp4", w, words, scales)
    n, k = (int(v) for v in w.shape)
    if w.dtype != torch.bfloat16 or w.stride(-1) != 1:
        raise ValueError("quantize_fp4: the weight must be bfloat16 with contiguous rows")
    if words.shape != (n, k // 8) or scales.shape != (n, k // group_size) or scales.dtype != torch.uint8:
        raise ValueError("quantize_fp4: output shapes do not match the weight")
    _call("kx_quantize_fp4_bf16", _ptr(w), w.stride(0), _ptr(words), _ptr(scales), n, k, group_size, scale_kind,
          _stream())


def launch_quantize_mxfp8(w, words, scales, *, group_size: int = 32) -> None:
    """mxfp8 (words, scales) <- bf16 weight w (n, k) with contiguous rows."""
    _check_gpu("quantize_mxfp8", w, words, scales)
    n, k = (int(v) for v in w.shape)
    if w.dtype != torch.bfloat16 or w.stride(-1) != 1:
        raise ValueError("quantize_mxfp8: the weight must be bfloat16 with contiguous rows")
    if words.shape != (n, k // 4) or scales.shape != (n, k // group_size) or scales.dtype != torch.uint8:
        raise ValueError("quantize_mxfp8: output shapes do not match the weight")
    _call("kx_quantize_mxfp8_bf16", _ptr(w), w.stride(0), _ptr(words), _ptr(scales), n, k, group_size, _stream())


def launch_tile_weights(words, scales, biases, wt, sbt, *, n, k, group_size, bits) -> None:
    _check_gpu("tile_weights", words, scales, biases, wt, sbt)
    _call(
        "kx_qweight_tile_affine", _ptr(words), _ptr(scales), _ptr(biases), _ptr(wt), _ptr(sbt), n, k,
        group_size, bits, _stream(),
    )


def launch_qgemm_tiled(a, wt, sbt, out, *, n, k, bits, bias=None, flags: int = 0, resid=None,
                       gate=None) -> None:
    _check_gpu("qgemm_tiled", a, wt, sbt, out, bias, resid, gate)
    flags |= _dtype_flags(out, resid, "quantized linear")
    m, ka, lda = _rows(a, "quantized linear input")
    if ka != k:
        raise ValueError(f"quantized linear: input width {ka} does not match {k}")
    _, _, ldc = _rows(out, "quantized linear output")
    ldr, div, stride = 0, 1, 0
    if resid is not None:
        _, _, ldr = _rows(resid, "quantized linear residual")
        div, stride = _mod_rows(gate, m, n, "quantized linear gate")
    _call(
        "kx_qgemm_affine_tiled_bf16", _ptr(a), lda, _ptr(wt), _ptr(sbt), _ptr(bias), _ptr(out), ldc, m,
        n, k, bits, flags, _ptr(resid), ldr, _ptr(gate), div, stride, _stream(),
    )


def launch_dequant(words, scales, biases, out, *, n, k, group_size, bits) -> None:
    _check_gpu("dequant", words, scales, biases, out)
    _call(
        "kx_dequant_affine_bf16", _ptr(words), _ptr(scales), _ptr(biases), _ptr(out), n, k,
        group_size, bits, _stream(),
    )


def launch_unary(name: str, x, out) -> None:
    """``name``: the entry point without its type suffix (``kx_gelu_tanh``, ``kx_silu``)."""
    _check_gpu(name, x, out)
    sfx = _suffix(x, name)
    _same_dtype(name, x.dtype, out)
    if not (x.is_contiguous() and out.is_contiguous()):
        raise ValueError(f"{name}: contiguous tensors required")
    _call(f"{name}_{sfx}", _ptr(x), _ptr(out), x.numel(), _stream())


def launch_swiglu(x, out) -> None:
    _check_gpu("swiglu", x, out)
    sfx = _suffix(x, "swiglu")
    _same_dtype("swiglu", x.dtype, out)
    rows, width, ldx = _rows(x, "swiglu x")
    _, _, ldy = _rows(out, "swiglu out")
    _call(f"kx_swiglu_{sfx}", _ptr(x), ldx, _ptr(out), ldy, rows, width // 2, _stream())


def launch_modulate(x, out, shift, scale) -> None:
    _check_gpu("modulate", x, out, shift, scale)
    sfx = _suffix(x, "modulate")
    _same_dtype("modulate", x.dtype, out)
    rows, dim, ldx = _rows(x, "modulate x")
    _, _, ldy = _rows(out, "modulate out")
    div, stride = _shared_mod_rows(shift, scale, rows, dim, "modulate")
    _call(
        f"kx_modulate_{sfx}", _ptr(x), ldx, _ptr(out), ldy, rows, dim, _ptr(shift), _ptr(scale),
        div, stride, _stream(),
    )


def table_add(table: torch.Tensor, ts: torch.Tensor | None, round_to: torch.dtype = torch.float32) -> torch.Tensor:
    """``fp32(table) + fp32(ts)`` as a new contiguous fp32 ``(B, T, rows, D)`` tensor: ``table`` is
    ``(rows, D)`` (fp32, bf16 or fp16), ``ts`` ``(B, T, rows, D)`` with a contiguous last axis (other
    strides may be 0 to broadcast), or ``None`` (the table alone, as ``(1, 1, rows, D)``). With
    ``round_to`` bf16 or fp16 every sum is rounded to that type (and kept as fp32)."""
    _check_gpu("table_add", table, ts)
    if table.dim() != 2 or table.stride(-1) != 1 or (table.shape[0] > 1 and table.stride(0) != table.shape[1]):
        raise ValueError("table_add: table must be a contiguous (rows, dim) tensor")
    rows, dim = table.shape
    if ts is None:
        batch, tokens, bs, tstride, rs, ts_code = 1, 1, 0, 0, 0, KX_F32
    else:
        if ts.dim() != 4 or ts.shape[2:] != (rows, dim) or ts.stride(-1) != 1:
            raise ValueError(f"table_add: timestep modulation {tuple(ts.shape)} does not match table {(rows, dim)}")
        batch, tokens = ts.shape[:2]
        bs, tstride, rs = ts.stride(0), ts.stride(1), ts.stride(2)
        ts_code = _weight_code(ts, "table_add timestep")
    round_code = {torch.float32: KX_F32, torch.bfloat16: KX_BF16, torch.float16: KX_F16}.get(round_to)
    if round_code is None:
        raise ValueError(f"table_add: round_to must be float32, bfloat16 or float16, got {round_to}")
    out = torch.empty((batch, tokens, rows, dim), dtype=torch.float32, device=table.device)
    _call("kx_table_add_f32", _ptr(table), _weight_code(table, "table_add table"), _ptr(ts), ts_code, bs, tstride, rs,
          _ptr(out), batch, tokens, rows, dim, round_code, _stream())
    return out


def launch_gated_residual(x, r, out, gate) -> None:
    _check_gpu("gated_residual", x, r, out, gate)
    sfx = _suffix(r, "gated_residual")
    _same_dtype("gated_residual", r.dtype, x, out)
    rows, dim, ldr = _rows(r, "gated_residual residual")
    ldx = 0
    if x is not None:
        _, _, ldx = _rows(x, "gated_residual x")
    _, _, ldy = _rows(out, "gated_residual out")
    div, stride = _mod_rows(gate, rows, dim, "gated_residual gate")
    _call(
        f"kx_gated_residual_{sfx}", _ptr(x), ldx, _ptr(r), ldr, _ptr(out), ldy, rows, dim, _ptr(gate),
        div, stride, _stream(),
    )


def _dtype_code(t, name: str) -> int:
    if t.dtype == torch.float32:
        return KX_F32
    if t.dtype == torch.bfloat16:
        return KX_BF16
    raise ValueError(f"{name}: tensors must be bfloat16 or float32, got {t.dtype}")


def _dense(name: str, *tensors) -> None:
    _check_gpu(name, *tensors)
    for t in tensors:
        if t is not None and not t.is_contiguous():
            raise ValueError(f"{name}: tensors must be contiguous")


def launch_timestep_embedding(t, out, neg_log_period: float, time_scale: float = 1.0) -> None:
    """out (n, dim) fp32 or bf16 <- sinusoidal features of the fp32 timesteps t (n,) * time_scale."""
    _dense("timestep_embedding", t, out)
    if t.dtype != torch.float32 or t.dim() != 1 or out.dim() != 2 or out.shape[0] != t.shape[0]:
        raise ValueError("timestep_embedding: t must be fp32 (n,) and out (n, dim)")
    _call("kx_timestep_embedding", _ptr(t), _ptr(out), t.shape[0], out.shape[1],
          _dtype_code(out, "timestep_embedding"), time_scale, neg_log_period, _stream())


def launch_ltx_rope_tables(positions, max_pos, grid, cos, sin, *, middle: bool) -> None:
    """cos, sin (B, T, half) fp32 <- LTX split-RoPE angles of fp32 positions (B, axes, T[, 2])."""
    _dense("ltx_rope_tables", positions, max_pos, grid, cos, sin)
    if any(t.dtype != torch.float32 for t in (positions, max_pos, grid, cos, sin)):
        raise ValueError("ltx_rope_tables: every tensor is float32")
    batch, axes, tokens = (int(s) for s in positions.shape[:3])
    stride = int(positions.shape[3]) if positions.dim() == 4 else 1
    half = int(cos.shape[-1])
    if cos.shape != (batch, tokens, half) or sin.shape != cos.shape or max_pos.numel() != axes:
        raise ValueError("ltx_rope_tables: table or max_pos shape does not match the positions")
    _call("kx_ltx_rope_tables", _ptr(positions), stride, int(middle), _ptr(max_pos), _ptr(grid), _ptr(cos),
          _ptr(sin), batch, axes, tokens, grid.numel(), half, _stream())


def launch_euler_velocity_step(sample, velocity, out, delta: float) -> None:
    _dense("euler_velocity_step", sample, velocity, out)
    if not (sample.shape == velocity.shape == out.shape) or not (sample.dtype == velocity.dtype == out.dtype):
        raise ValueError("euler_velocity_step: sample, velocity and out must share shape and dtype")
    _call("kx_euler_velocity_step", _ptr(sample), _ptr(velocity), _ptr(out), sample.numel(),
          _dtype_code(sample, "euler_velocity_step"), delta, _stream())


def launch_euler_step(sample, denoised, out, ratio: float) -> None:
    _dense("euler_step", sample, denoised, out)
    if not (sample.shape == denoised.shape == out.shape) or out.dtype != sample.dtype:
        raise ValueError("euler_step: shapes must match and out must have the sample dtype")
    _call("kx_euler_step", _ptr(sample), _dtype_code(sample, "euler_step"), _ptr(denoised),
          _dtype_code(denoised, "euler_step"), _ptr(out), sample.numel(), ratio, _stream())


def launch_to_denoised(latent, velocity, timesteps, out, *, rows: int, dim: int, ts_div: int) -> None:
    _dense("to_denoised", latent, velocity, timesteps, out)
    if timesteps.dtype != torch.float32 or latent.numel() != rows * dim or velocity.numel() != rows * dim \
            or out.numel() != rows * dim or out.dtype != latent.dtype or timesteps.numel() * ts_div != rows:
        raise ValueError("to_denoised: shapes or dtypes do not match")
    _call("kx_to_denoised", _ptr(latent), _dtype_code(latent, "to_denoised"), _ptr(velocity),
          _dtype_code(velocity, "to_denoised"), _ptr(timesteps), _ptr(out), rows, dim, ts_div, _stream())


def launch_mask_composite(denoised, clean, mask, out, *, rows: int, dim: int) -> None:
    _dense("mask_composite", denoised, clean, mask, out)
    if mask.dtype != torch.float32 or mask.numel() != rows or denoised.numel() != rows * dim \
            or clean.numel() != rows * dim or out.numel() != rows * dim or out.dtype != denoised.dtype:
        raise ValueError("mask_composite: shapes or dtypes do not match")
    _call("kx_mask_composite", _ptr(denoised), _dtype_code(denoised, "mask_composite"), _ptr(clean),
          _dtype_code(clean, "mask_composite"), _ptr(mask), _ptr(out), rows, dim, _stream())


def launch_all_finite(x, flag) -> None:
    """flag (one int32 on the device) <- 1 when every element of x is finite, else 0."""
    _dense("all_finite", x, flag)
    if flag.dtype != torch.int32 or flag.numel() < 1:
        raise ValueError("all_finite: flag must be an int32 device tensor")
    _call("kx_all_finite", _ptr(x), x.numel(), _dtype_code(x, "all_finite"), _ptr(flag), _stream())


def launch_quantize(w, words, scales, biases, *, group_size: int, bits: int) -> None:
    """Packed affine (words, scales, biases) <- bf16 weight w (n, k) with contiguous rows."""
    _check_gpu("quantize_affine", w, words, scales, biases)
    n, k = (int(v) for v in w.shape)
    if w.dtype != torch.bfloat16 or w.stride(-1) != 1:
        raise ValueError("quantize_affine: the weight must be bfloat16 with contiguous rows")
    if words.shape != (n, k * bits // 32) or scales.shape != (n, k // group_size) or biases.shape != scales.shape:
        raise ValueError("quantize_affine: output shapes do not match the weight")
    _call("kx_quantize_affine_bf16", _ptr(w), w.stride(0), _ptr(words), _ptr(scales), _ptr(biases), n, k,
          group_size, bits, _stream())
