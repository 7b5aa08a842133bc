"""Model-level integration: kernel attention for the experiment models, over the fused additive layers.

The reference's experiments (Experiments/kernel_attention) reach the weighted abs / Laplace sums through three
entries, provided here with the same names and arguments:

  * attention(q, k, v, kernel, tau, keep=None, impl="efficient") (attention.py:95-126), on (B, H, S, D) fp32
    tensors; keep (B, S) marks the real keys. The additive kernels (add_laplace, add_riesz, add_bump) run as one
    fused libqlka call each (qlka.layers); "softmax" is scaled dot-product attention with scale tau**-2
    (attention.py:99-102). TAU holds the default temperatures (kernels.py:13-25).
  * KernelMultiheadAttention(embed_dim, num_heads, kernel, tau, impl) (vision_transformer.py:19-44): self-attention
    whose state_dict is nn.MultiheadAttention's (in_proj_weight, in_proj_bias, out_proj), so trained weights load.
  * use_kernel_attention(model, kernel, tau, impl) and KernelAttention(config, kernel, tau, impl) (nomic.py:9-40):
    kernel attention inside a HF NomicBertModel with its own weights.

The nomic integration goes through transformers' attention-function registry instead of replacing modules: the
registry entry "qlka" is an attention function (q, k, v after the layer's projections and rotary embedding, in
(B, H, S, D)) that reads the kernel from the calling attention module, and the model's attention implementation is
switched to it. The layers keep their own NomicBertAttention objects and parameters; the key mask is the boolean
SDPA-style mask the model builds for "sdpa" (the same mask builder is registered for "qlka").
"""

import copy

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import layers

TAU = {"softmax": 64 ** 0.25, "add_laplace": 0.5, "add_riesz": 1.0, "add_bump": 1.5}   # kernels.py:13-25
KERNELS = tuple(TAU)
IMPLS = ("naive", "efficient")


def _softmax(q, k, v, tau, keep):
    mask = None if keep is None else keep.bool()[:, None, None, :]
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=tau ** -2)


def attention(q, k, v, kernel, tau, keep=None, impl="efficient"):
    """Kernel attention of (B, H, S, D) fp32 q, k, v; keep (B, S), nonzero = real key, or None."""
    assert q.dtype == k.dtype == v.dtype == torch.float32, "kernel attention runs in fp32 only"
    assert impl in IMPLS, f"impl must be one of {IMPLS}"
    if kernel == "softmax":
        return _softmax(q, k, v, tau, keep)
    if kernel not in layers.LAYERS:
        raise NotImplementedError(f"kernel {kernel!r} does not run on the weighted abs / Laplace sums; "
                                  f"available: {sorted(KERNELS)}")
    if impl == "naive":
        raise NotImplementedError("impl='naive' (the dense kernel matrix) is not part of this package; "
                                  "use impl='efficient'")
    return layers.attention(q, k, v, kernel, tau, keep)


def _resolve_tau(kernel, tau):
    if tau is not None:
        return float(tau)
    if kernel not in TAU:
        raise NotImplementedError(f"kernel {kernel!r} has no default temperature; available: {sorted(KERNELS)}")
    return TAU[kernel]


# --------------------------------------------------------------------------------------------- vision transformer
class KernelMultiheadAttention(nn.Module):
    """x (B, S, E) -> (B, S, E) self-attention with a chosen kernel. Parameters and their initialisation follow
    nn.MultiheadAttention (packed q/k/v input projection, output projection), so its state_dict loads both ways."""

    def __init__(self, embed_dim, num_heads, kernel="softmax", tau=None, impl="efficient"):
        super().__init__()
        if embed_dim % num_heads:
            raise ValueError(f"embed_dim {embed_dim} is not a multiple of num_heads {num_heads}")
        self.num_heads = num_heads
        self.kernel, self.tau, self.impl = kernel, _resolve_tau(kernel, tau), impl
        self.in_proj_weight = nn.Parameter(nn.init.xavier_uniform_(torch.empty(3 * embed_dim, embed_dim)))
        self.in_proj_bias = nn.Parameter(torch.zeros(3 * embed_dim))
        self.out_proj = nn.Linear(embed_dim, embed_dim)
        nn.init.xavier_uniform_(self.out_proj.weight)
        nn.init.zeros_(self.out_proj.bias)

    def split_heads(self, x):
        """The packed projection of x as three (B, H, S, E / H) tensors q, k, v."""
        packed = F.linear(x, self.in_proj_weight, self.in_proj_bias)            # [q | k | v] along the last dim
        per_head = packed.unflatten(-1, (3, self.num_heads, -1))                 # (B, S, 3, H, Dh)
        return per_head.permute(2, 0, 3, 1, 4).unbind(0)

    def forward(self, x, keep=None):
        q, k, v = self.split_heads(x)
        heads = attention(q, k, v, self.kernel, self.tau, keep, self.impl)      # (B, H, S, Dh)
        return self.out_proj(heads.transpose(1, 2).flatten(2))


# ---------------------------------------------------------------------------------------------------- nomic-bert
REGISTRY_NAME = "qlka"
_registered = False


def _hf_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """transformers attention function: (B, H, S, D) states of one layer -> ((B, S, H, D) output, None). The kernel
    is the one use_kernel_attention / KernelAttention attached to the layer's attention module."""
    kernel, tau, impl = module.qlka_kernel
    keep = None
    if attention_mask is not None:
        if attention_mask.dtype != torch.bool:
            raise TypeError("kernel attention expects the boolean key mask of the sdpa mask builder")
        keep = attention_mask[:, 0, 0, :]            # every query row of the bidirectional mask holds the key mask
    out = attention(query.contiguous(), key.contiguous(), value.contiguous(), kernel, tau, keep, impl)
    return out.transpose(1, 2), None


def register():
    """Register the "qlka" attention function (and the sdpa boolean-mask builder under the same name) with
    transformers. Idempotent."""
    global _registered
    if _registered:
        return REGISTRY_NAME
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask
    AttentionInterface.register(REGISTRY_NAME, _hf_attention)
    AttentionMaskInterface.register(REGISTRY_NAME, sdpa_mask)
    _registered = True
    return REGISTRY_NAME


def _tag(attn, kernel, tau, impl):
    if impl not in IMPLS:
        raise ValueError(f"impl must be one of {IMPLS}")
    attn.qlka_kernel = (kernel, _resolve_tau(kernel, tau), impl)
    attn.kernel, attn.tau, attn.impl = attn.qlka_kernel


def _encoder(model):
    """The NomicBertModel of a model: the model itself, or the auto_model of a SentenceTransformer's first module."""
    if hasattr(model, "layers"):
        return model
    return model[0].auto_model


def use_kernel_attention(model, kernel, tau=None, impl="efficient"):
    """Run every attention layer of a NomicBertModel (or a SentenceTransformer wrapping one) with `kernel`, in place;
    every parameter stays where it is. Returns the model."""
    name = register()
    enc = _encoder(model)
    for layer in enc.layers:
        _tag(layer.self_attn, kernel, tau, impl)
    enc.set_attn_implementation(name)
    return model


def KernelAttention(config, kernel="softmax", tau=None, impl="efficient"):
    """A NomicBertAttention for `config` (same parameters: q_proj, k_proj, v_proj, o_proj) that runs `kernel`; its
    config is a copy with the attention implementation set to the registered kernel attention."""
    from transformers.models.nomic_bert.modeling_nomic_bert import NomicBertAttention
    cfg = copy.copy(config)
    cfg._attn_implementation = register()
    attn = NomicBertAttention(cfg)
    _tag(attn, kernel, tau, impl)
    return attn
