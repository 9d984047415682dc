"""MI355X-native SmolVLA bf16 inference hot path.

* ``smolvla.ops``      -- torch wrappers over the C-ABI of ``libsvla.so``
* ``smolvla.kernels``  -- the reference's per-kernel harness names
* ``smolvla.vla``      -- the reference's layer-module signatures
* ``smolvla.pipeline`` -- the full chunk engine (vision -> prefix -> 10 Euler steps)
"""

from .config import DecoderConfig, SmolVLAConfig, VitConfig, small_config  # noqa: F401

__version__ = "0.1.0"
