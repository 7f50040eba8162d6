"""elsa_amd: MI355X-native (gfx950) ELSA two-pass exact monoid-scan attention.

Public names follow the reference package (reference ``__init__.py:1-21``).  Device
work runs in ``libelsa_hip.so`` (hand-written HIP kernels behind a C ABI,
``include/elsa_hip.h``), loaded through ctypes; there is no Triton or CPU fallback.
"""
from .attention import twopass_attention
from .attention_bwd import twopass_attention_backward, twopass_attention_train, twopass_attention_with_state
from .full_model import TransformerEncoder, make_model_pair
from .full_model_bwd import TrainableTransformerEncoder, make_train_model_pair
from .timm_dropin import PatchReport, patch_timm_attention
from .timm_dropin_bwd import TrainPatchReport, patch_timm_attention_train

__all__ = [
    "PatchReport",
    "TrainPatchReport",
    "TransformerEncoder",
    "TrainableTransformerEncoder",
    "make_model_pair",
    "make_train_model_pair",
    "patch_timm_attention",
    "patch_timm_attention_train",
    "twopass_attention",
    "twopass_attention_backward",
    "twopass_attention_train",
    "twopass_attention_with_state",
]
