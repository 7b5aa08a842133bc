"""Model-level integration: the attention modules of Experiments/kernel_attention over the fused additive layers.

Mirrors, with the same names, parameters and call conventions:
  * attention(q, k, v, kernel, tau, keep=None, impl="efficient") (attention.py:95-126) for the kernels that run on
    the weighted abs / Laplace sums (add_laplace, add_riesz, add_bump, through qlka.layers) and for "softmax"
    (scaled dot-product attention with scale tau**-2, attention.py:99-102). The reference's other kernels (gauss,
    laplace, riesz, tri, elu, relu, dpfp) never call these operators and are not provided here.
  * TAU, the default temperatures of those kernels (kernels.py:13-25).
  * KernelMultiheadAttention (vision_transformer.py:19-44): self-attention with the parameters of
    nn.MultiheadAttention (in_proj_weight, in_proj_bias, out_proj), so its weights load unchanged.
  * KernelAttention and use_kernel_attention (nomic.py:9-40): a NomicBertAttention whose scaled dot-product is
    replaced by the kernel attention, taking its key mask from the boolean mask the model builds for SDPA.
"""

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import layers

TAU = {"softmax": 64 ** 0.25, "add_laplace": 0.5, "add_riesz": 1.0, "add_bump": 1.5}   # kernels.py:13-25
KERNELS = tuple(TAU)


def attention(q, k, v, kernel, tau, keep=None, impl="efficient"):
    """q, k, v (B, H, S, D) fp32 -> (B, H, S, D); keep (B, S) marks the real keys (attention.py:95-126)."""
    assert q.dtype == k.dtype == v.dtype == torch.float32, "kernel attention runs in fp32 only"
    assert impl in ("naive", "efficient")
    if kernel == "softmax":
        mask = None if keep is None else keep[:, None, None, :].bool()
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=tau ** -2)
    if kernel not in layers.LAYERS:
        raise NotImplementedError(f"kernel {kernel!r} does not run on the weighted abs / Laplace sums; "
                                  f"available: {sorted(KERNELS)}")
    if impl != "efficient":
        raise NotImplementedError("impl='naive' (the dense kernel matrix) is not part of this package; "
                                  "use impl='efficient'")
    return layers.attention(q, k, v, kernel, tau, keep)


class KernelMultiheadAttention(nn.Module):
    """Self-attention with a pluggable kernel; parameter-compatible with nn.MultiheadAttention
    (vision_transformer.py:19-44). x (B, S, E) -> (B, S, E)."""

    def __init__(self, embed_dim, num_heads, kernel="softmax", tau=None, impl="efficient"):
        super().__init__()
        assert embed_dim % num_heads == 0
        self.num_heads = num_heads
        self.head_dim = embed_dim // num_heads
        self.kernel = kernel
        self.tau = TAU[kernel] if tau is None else tau
        self.impl = impl
        self.in_proj_weight = nn.Parameter(torch.empty(3 * embed_dim, embed_dim))
        self.in_proj_bias = nn.Parameter(torch.empty(3 * embed_dim))
        self.out_proj = nn.Linear(embed_dim, embed_dim)
        nn.init.xavier_uniform_(self.in_proj_weight)
        nn.init.zeros_(self.in_proj_bias)
        nn.init.xavier_uniform_(self.out_proj.weight)
        nn.init.zeros_(self.out_proj.bias)

    def forward(self, x, keep=None):
        B, S, E = x.shape
        proj = F.linear(x, self.in_proj_weight, self.in_proj_bias)                           # (B, S, 3E)
        q, k, v = proj.view(B, S, 3, self.num_heads, self.head_dim).permute(2, 0, 3, 1, 4)   # 3 x (B, H, S, D)
        out = attention(q, k, v, self.kernel, self.tau, keep, self.impl)
        return self.out_proj(out.transpose(1, 2).reshape(B, S, E))


def _nomic_attention_base():
    from transformers.models.nomic_bert.modeling_nomic_bert import NomicBertAttention, apply_rotary_pos_emb
    return NomicBertAttention, apply_rotary_pos_emb


def _kernel_attention_class():
    NomicBertAttention, apply_rotary_pos_emb = _nomic_attention_base()

    class KernelAttention(NomicBertAttention):
        """NomicBertAttention with a pluggable kernel and the same parameters (nomic.py:9-31)."""

        def __init__(self, config, kernel="softmax", tau=None, impl="efficient"):
            super().__init__(config)
            self.kernel = kernel
            self.tau = TAU[kernel] if tau is None else tau
            self.impl = impl

        def forward(self, hidden_states, attention_mask=None, position_embeddings=None, **kwargs):
            B, S, _ = hidden_states.shape
            shape = (B, S, -1, self.head_dim)
            q = self.q_proj(hidden_states).view(shape).transpose(1, 2)            # (B, H, S, D)
            k = self.k_proj(hidden_states).view(shape).transpose(1, 2)
            v = self.v_proj(hidden_states).view(shape).transpose(1, 2)
            q, k = apply_rotary_pos_emb(q, k, *position_embeddings)
            keep = None
            if attention_mask is not None:
                # the SDPA-style mask is boolean and every row holds the key-keep pattern
                if attention_mask.dtype != torch.bool:
                    raise TypeError("expected a boolean attention mask (attn_implementation='sdpa')")
                keep = attention_mask[:, 0, 0, :]
            out = attention(q.contiguous(), k.contiguous(), v.contiguous(), self.kernel, self.tau, keep, self.impl)
            return self.o_proj(out.transpose(1, 2).reshape(B, S, -1)), None

    return KernelAttention


_KERNEL_ATTENTION = None


def KernelAttention(config, kernel="softmax", tau=None, impl="efficient"):
    """Construct the nomic KernelAttention module (the class needs transformers, imported on first use)."""
    global _KERNEL_ATTENTION
    if _KERNEL_ATTENTION is None:
        _KERNEL_ATTENTION = _kernel_attention_class()
    return _KERNEL_ATTENTION(config, kernel, tau, impl)


def use_kernel_attention(model, kernel, tau=None, impl="efficient"):
    """Swap every attention layer in place, keeping its weights (nomic.py:34-40). `model` is a NomicBertModel or a
    SentenceTransformer whose first module wraps one (model[0].auto_model)."""
    auto = model if hasattr(model, "layers") else model[0].auto_model
    for layer in auto.layers:
        new = KernelAttention(auto.config, kernel, tau, impl).to(layer.self_attn.q_proj.weight.device)
        new.load_state_dict(layer.self_attn.state_dict())
        layer.self_attn = new
    return model
