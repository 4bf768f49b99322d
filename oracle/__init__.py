"""CPU oracle for the DiT-block hot path: TEST INFRASTRUCTURE, not product code.

A numpy restatement of the reference's (dmlsrc/KinoMLX) MLX math for the diffusion-transformer
block: modulated norms, RoPE, attention, linear layers, the affine int4/int8 weight format and
the block compositions; and the steps either side of the block (timestep features, AdaLN
modulation producers, the output head, the transformer forward, the X0 conversion, the
conditioning composite, the Euler updates and the finite check, ``oracle/denoise.py``). Every function cites the reference file:line it follows (paths are
relative to the reference checkout).

``oracle/torch_cpu.py`` restates the config-1 block once more in FP32 on torch's CPU kernels: the
timed CPU baseline, pinned to the numpy restatement.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker or the timed CPU baseline. The product package
``kinomlx_amd`` never imports it: there is no CPU fallback on the product path.

Arithmetic policy: float32 opmath throughout (the "fp32 evaluation" the parity tolerances are
stated against), with bfloat16 values carried as float32 arrays holding bf16-representable
numbers. The int4/int8 dequantisation is restated bit-exactly (fp32 ``scale*q + bias`` then one
round-to-nearest-even into bf16).

Pinning: each function is checked by ``tests/test_oracle.py`` against the reference's own
known-answer tests where they exist (the RoPE frequency grid of
``tests/models/ltx2/transformer/test_primitives.py:115-132`` and the Krea axis-order test of
``tests/models/krea2/transformer/test_transformer.py:302-327``; the Euler, X0 and composite
known answers of ``tests/samplers/test_steps.py:10-71``,
``tests/models/ltx2/transformer/test_model.py:572-594``, ``tests/models/ltx2/test_state.py:99-124``
and ``tests/models/ltx2/test_denoise.py:36-67``), the committed vectors under
``tests/golden/``, and float64 / closed-form checks chosen so that a dropped term, a wrong sign or
index, or a transposed operand fails.
"""

from .ops import *  # noqa: F401,F403
from .ops import __all__ as _ops_all
from .blocks import *  # noqa: F401,F403
from .blocks import __all__ as _blocks_all
from .denoise import *  # noqa: F401,F403
from .denoise import __all__ as _denoise_all

__all__ = list(_ops_all) + list(_blocks_all) + list(_denoise_all)
