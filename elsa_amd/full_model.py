"""Toy pre-norm Transformer encoders whose attention core switches between the ELSA two-pass
path and PyTorch's SDPA, for model-level comparisons of the two.

Public surface kept from the reference package (``__init__.py:1-21``): ``TransformerEncoder``
and ``make_model_pair`` here, the trainable variants in ``full_model_bwd``.  The constructor
keywords (``dim, depth, heads, mlp_ratio, backend, sdpa_kind, is_causal, elsa_kwargs``) and the
pair contract -- an SDPA baseline and an ELSA twin with identical weights (reference
``full_model.py:162-191``) -- are the reference's interface.  The modules are this
package's own: each layer has one fused qkv projection whose ``[B, N, 3, H, D]`` output the
ELSA core reads in place as strided q/k/v views and answers with ``[B, N, H, D]`` memory, so
no transposing copy is made on either side of the attention; the pair is the baseline and a
deep copy of it with its cores switched to ELSA.
"""
from __future__ import annotations

import copy
from typing import Literal, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from .attention_bwd import qkv_attention_train
from .timm_dropin import _attend

AttentionBackend = Literal["elsa", "sdpa"]
SdpaKind = Literal["auto", "math", "flash", "mem"]

_SDPA_KERNELS = {"math": SDPBackend.MATH, "flash": SDPBackend.FLASH_ATTENTION, "mem": SDPBackend.EFFICIENT_ATTENTION}


class AttentionCore(nn.Module):
    """Attention over a fused projection: ``[B, N, 3, H, D] -> [B, N, H*D]``; no parameters.

    ``elsa``: ``twopass_attention`` on strided views of the projection, or, when the core is
    ``trainable``, ``qkv_attention_train`` (forward with row state, exact-recompute backward,
    the projection's gradient written back in its own layout).  An inference core refuses
    inputs that need a gradient rather than cutting the graph.  ``sdpa``: PyTorch's
    ``scaled_dot_product_attention`` with the default or one pinned kernel (``sdpa_kind``).
    The softmax scale is 1/sqrt(head_dim) on both backends.
    """

    def __init__(self, backend: AttentionBackend, *, is_causal: bool = False, sdpa_kind: SdpaKind = "auto",
                 elsa_kwargs: Optional[dict] = None, trainable: bool = False) -> None:
        super().__init__()
        self.is_causal = bool(is_causal)
        self.trainable = bool(trainable)
        self.configure(backend, sdpa_kind=sdpa_kind, elsa_kwargs=elsa_kwargs)

    def configure(self, backend: AttentionBackend, *, sdpa_kind: SdpaKind = "auto",
                  elsa_kwargs: Optional[dict] = None) -> None:
        if backend not in ("elsa", "sdpa"):
            raise ValueError(f"unknown attention backend: {backend}")
        if sdpa_kind != "auto" and sdpa_kind not in _SDPA_KERNELS:
            raise ValueError(f"unknown SDPA kind: {sdpa_kind}")
        self.backend = backend
        self.sdpa_kind = sdpa_kind
        # the encoders always ask for the paper-scan algorithm, the only one there is
        self.elsa_kwargs = {**(elsa_kwargs or {}), "algorithm": "paper_scan"}

    def forward(self, qkv: torch.Tensor) -> torch.Tensor:
        b, n, _, h, d = qkv.shape
        if self.backend == "elsa" and self.trainable:
            y = qkv_attention_train(qkv, is_causal=self.is_causal, **self.elsa_kwargs)
        else:
            q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
            if self.backend == "sdpa":
                y = self._sdpa(q, k, v)
            else:
                if torch.is_grad_enabled() and qkv.requires_grad:
                    raise RuntimeError("this encoder's ELSA attention is inference-only: use "
                                       "TrainableTransformerEncoder (twopass_attention_train) for gradients")
                y = _attend(q, k, v, {**self.elsa_kwargs, "is_causal": self.is_causal})
        return y.transpose(1, 2).reshape(b, n, h * d)

    def _sdpa(self, q, k, v):
        def call():
            return F.scaled_dot_product_attention(q, k, v, is_causal=self.is_causal, scale=q.shape[-1] ** -0.5)

        if self.sdpa_kind == "auto":
            return call()
        with sdpa_kernel(_SDPA_KERNELS[self.sdpa_kind]):
            return call()


class EncoderLayer(nn.Module):
    """``x + proj(attn(ln1(x)))``, then ``x + fc2(gelu(fc1(ln2(x))))``."""

    def __init__(self, dim: int, heads: int, hidden: int, core: AttentionCore) -> None:
        super().__init__()
        self.heads = heads
        self.norm1 = nn.LayerNorm(dim)
        self.qkv = nn.Linear(dim, 3 * dim)
        self.core = core
        self.proj = nn.Linear(dim, dim)
        self.norm2 = nn.LayerNorm(dim)
        self.fc1 = nn.Linear(dim, hidden)
        self.fc2 = nn.Linear(hidden, dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        b, n, c = x.shape
        qkv = self.qkv(self.norm1(x)).view(b, n, 3, self.heads, c // self.heads)
        x = x + self.proj(self.core(qkv))
        return x + self.fc2(F.gelu(self.fc1(self.norm2(x))))


class TransformerEncoder(nn.Module):
    """``depth`` pre-norm layers and a final LayerNorm over ``[B, N, dim]`` tokens."""

    trainable = False

    def __init__(self, *, dim: int = 192, depth: int = 1, heads: int = 3, mlp_ratio: float = 4.0,
                 backend: AttentionBackend, sdpa_kind: SdpaKind = "auto", is_causal: bool = False,
                 elsa_kwargs: Optional[dict] = None) -> None:
        super().__init__()
        if dim % heads != 0:
            raise ValueError("dim must be divisible by heads")
        hidden = int(round(dim * mlp_ratio))
        self.layers = nn.ModuleList(
            EncoderLayer(dim, heads, hidden, AttentionCore(backend, is_causal=is_causal, sdpa_kind=sdpa_kind,
                                                           elsa_kwargs=elsa_kwargs, trainable=self.trainable))
            for _ in range(depth))
        self.norm = nn.LayerNorm(dim)

    def set_attention(self, backend: AttentionBackend, *, sdpa_kind: SdpaKind = "auto",
                      elsa_kwargs: Optional[dict] = None) -> "TransformerEncoder":
        """Switch every layer's attention core (weights untouched); returns self."""
        for layer in self.layers:
            layer.core.configure(backend, sdpa_kind=sdpa_kind, elsa_kwargs=elsa_kwargs)
        return self

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for layer in self.layers:
            x = layer(x)
        return self.norm(x)


def _twin(baseline: TransformerEncoder, elsa_kwargs: Optional[dict]):
    """(baseline, its deep copy on ELSA): the same weights by construction."""
    return baseline, copy.deepcopy(baseline).set_attention("elsa", elsa_kwargs=elsa_kwargs)


def make_model_pair(*, dim: int = 192, depth: int = 1, heads: int = 3, mlp_ratio: float = 4.0,
                    sdpa_kind: SdpaKind = "auto", is_causal: bool = False,
                    elsa_kwargs: Optional[dict] = None) -> tuple[TransformerEncoder, TransformerEncoder]:
    """(SDPA baseline, ELSA) encoders with identical weights."""
    baseline = TransformerEncoder(dim=dim, depth=depth, heads=heads, mlp_ratio=mlp_ratio, backend="sdpa",
                                  sdpa_kind=sdpa_kind, is_causal=is_causal)
    return _twin(baseline, elsa_kwargs)
