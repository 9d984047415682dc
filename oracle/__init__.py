"""CPU oracle for the SmolVLA bf16 inference hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (``vla-to-npu_amd/``)
imports this package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker or as
the timed CPU baseline, never as the thing measured or shipped.

The oracle restates, in PyTorch on the CPU, the reference's own PyTorch
reference modules (the parity target named by the task):

* ``TextEncoderBlock``           vla/text_encoder_bf16.py:61-135
* ``ActionExpertSelfBlock``      vla/action_expert_bf16.py:69-128
* ``ActionExpertCrossBlock``     vla/action_expert_bf16.py:134-207
* ``MiniVit``                    vla/vision_block_bf16.py:57-79
* ``preproc_ref`` / ``con_ref``  vla/vla.py:396-408, 434-437
* ``postprocessing_ref``         vla/vla.py:506-516
* SigLIP position embedding      vla/vit_emb.py:43-47

plus the pieces the reference does not have and the target configuration
adds (10-step Euler flow matching, sinusoidal time embedding, action in/out
projections, three cameras, the 241-token prefix with a prefix-LM mask).

Every function is pinned by tests in ``tests/test_oracle_*.py`` against an
independent implementation (torch functional ops, ``transformers``' Llama /
SigLIP / Idefics3 code built from local configs, closed forms, brute force).
No function here is "parity unpinned"; the header of each test file says
which check pins which function.
"""

from .smolvla_ref import *  # noqa: F401,F403
