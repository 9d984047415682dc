"""Reference-signature layer modules.

Same module and function names, argument order and weight layout (``[in, out]``,
``params`` keys) as the reference's ``vla/*_bf16.py`` layer files; each call
runs the gfx950 kernels of ``libsvla.so``.  Inputs may be CPU or GPU tensors
(``[S, H]`` like the reference's arrays, or batched ``[B, S, H]``); results are
returned on the input's device.
"""
