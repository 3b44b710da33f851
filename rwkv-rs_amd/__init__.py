"""MI355X-native WKV7 time-mix recurrence (forward, backward, decode) behind a
C ABI (include/wkv7.h) that mirrors rwkv-nn's Burn WKV7 operator traits.

* ``wkv7``      -- the operator API over torch device tensors (imports torch)
* ``synthetic`` -- seeded operands with the benchmark's value distributions
* ``build``     -- compiles libwkv7_hip.so for gfx950
* ``neighbors`` -- the fused ops on either side of the operator (token shift
  + channel mixes, gated readout; include/rwkv_neighbors.h)
* ``model``     -- an RWKV-7 language-model training step that calls ``wkv7``
* ``weights``   -- RWKV-7 release checkpoints (.pth) mapped onto ``model``
"""

import importlib

from . import synthetic  # noqa: F401


def __getattr__(name):
    if name in ("wkv7", "_native", "build", "model", "neighbors", "weights", "lm_loss"):
        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(name)
