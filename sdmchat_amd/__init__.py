"""sdmchat_amd -- the run-time SDM mixer (RunTimeSdm) of SDMCHAT on AMD MI355X (gfx950).

``RunTimeSdm``      drop-in nn.Module (same constructor, state_dict and forward signature as the reference's)
``TrainedSdm``      drop-in for the trained product-key table layer (same constructor and state_dict)
``OneSdmLM``        the whole language model around the mixer (same constructor and state_dict; no archive)
``core``            torch-facing wrappers of the C ABI (addressing, the SDM core)
``synthetic``       seeded synthetic parameters and inputs of the layer workloads
``DecodeGraph``, ``ForwardGraph``  OneSdmLM.step and OneSdmLM.forward at fixed shapes, captured in HIP graphs
``build``           compiles ``csrc/*.hip`` into ``lib/libsdm_rt.so``
"""
from .runtime_sdm import RMSNorm, RunTimeSdm  # noqa: F401
from .trained_sdm import TrainedSdm  # noqa: F401
from .model import DecodeGraph, ForwardGraph, ModelDecodeState, OneSdmLM, decode_state_bytes  # noqa: F401
