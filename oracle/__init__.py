"""CPU oracle for the muon_sr optimizer-step hot path.

TEST INFRASTRUCTURE ONLY: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or as the timed CPU baseline.  The product package ``muon_sr_amd`` never
imports it and has no CPU fallback.

Contents
--------
* ``oracle.c`` (built to ``oracle/_build/liboracle.so`` by ``oracle/Makefile``):
  Philox4x32-10, stochastic rounding, the 8-bit quantizer search and the five
  elementwise kernels, in strict IEEE binary32.
* :mod:`oracle.ref` (this package): ctypes bindings, bf16 helpers, the dynamic
  codebook, Newton-Schulz restatements and deterministic seeds.
* :mod:`oracle.torch_ref`: a torch transcription of the reference's
  pure-PyTorch optimizers, used as the host-core baseline.
"""
from .ref import *  # noqa: F401,F403
