"""muon_sr_amd: the muon_sr optimizer-step hot path on AMD MI355X (gfx950).

Drop-in replacements for bab2min/muon_sr 0.1.2's GPU optimizers
(``from muon_sr import TritonMuonSR`` -> ``from muon_sr_amd import TritonMuonSR``):
the classes below keep the reference's constructors, param-group keys, state
keys, seeds and checkpoint format, and run hand-written HIP kernels for
gfx950 through the C ABI of ``libmuon_sr_amd.so`` (include/muon_sr_amd.h).
"""
from ._version import __version__
from ._lib import set_sr_noise, get_sr_noise
from .adamw_8bit import TritonAdamW8bit, create_dynamic_map
from .adamw import TritonAdamW, TritonSRAccumulator
from .muon import TritonMuonSR, TritonMuonSRWithAuxAdam, newton_schulz
from .linear import SRLinear, linear_wgrad_sr_accum

__all__ = [
    "TritonAdamW8bit",
    "TritonAdamW", "TritonSRAccumulator",
    "TritonMuonSR", "TritonMuonSRWithAuxAdam",
    "newton_schulz", "create_dynamic_map", "set_sr_noise", "get_sr_noise",
    "SRLinear", "linear_wgrad_sr_accum",
]
