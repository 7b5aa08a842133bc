"""GPU parity of the model-level integration (qlka.modules, qlka.harness) with the additive kernels.

* KernelMultiheadAttention (vision_transformer.py:19-44): against the float64 normalised kernel matrix
  (kernels.py:68-89, restated in oracle/dense.py) over the module's own projections.
* nomic KernelAttention (nomic.py:9-40) inside NomicBertModel: the padding mask the model builds is the key mask, so
  the real tokens of a padded document get the hidden states of the same document run unpadded, and each layer's
  attention matches the float64 kernel matrix with that mask.
* The GPU-time harness (pareto.py:46-65 stand-in) runs end to end at a small size.
"""

import numpy as np
import pytest
import torch

from oracle import dense

pytestmark = pytest.mark.gpu

KERNELS = ("add_laplace", "add_riesz", "add_bump")


def _dense_attention(kernel, q, k, v, tau, keep=None):
    """(B, H, S, D) float64 normalised kernel-matrix attention (kernels.py:68-89, attention.py:31-34)."""
    B, H, S, D = q.shape
    P = B * H
    q64 = q.detach().cpu().double().transpose(2, 3).reshape(P, D, S)
    k64 = k.detach().cpu().double().transpose(2, 3).reshape(P, D, S)
    v64 = v.detach().cpu().double().reshape(P, S, -1)
    mask = None if keep is None else keep.cpu().repeat_interleave(H, dim=0).double()
    A = dense.dense_kernel_matrix(kernel, q64, k64, tau, mask)
    return ((A @ v64) / A.sum(dim=2, keepdim=True).clamp_min(dense.CLAMP)).view(B, H, S, -1)


@pytest.mark.parametrize("kernel", KERNELS)
def test_multihead_module_vs_float64(dev, kernel):
    from qlka import modules
    torch.manual_seed(2)
    E, H, B, S = 64, 4, 2, 150
    mod = modules.KernelMultiheadAttention(E, H, kernel=kernel).to(dev)
    x = torch.randn(B, S, E, device=dev)
    keep = torch.ones(B, S, dtype=torch.bool, device=dev)
    keep[1, 100:] = False
    with torch.no_grad():
        got = mod(x, keep)
        proj = torch.nn.functional.linear(x, mod.in_proj_weight, mod.in_proj_bias)
        q, k, v = proj.view(B, S, 3, H, E // H).permute(2, 0, 3, 1, 4)
        att = _dense_attention(kernel, q, k, v, mod.tau, keep)
        want = torch.nn.functional.linear(att.transpose(1, 2).reshape(B, S, E), mod.out_proj.weight.cpu().double(),
                                          mod.out_proj.bias.cpu().double())
    np.testing.assert_allclose(got.cpu().double().numpy(), want.numpy(), rtol=1e-4, atol=1e-5)


def _nomic(dev, kernel, layers=2, hidden=128, heads=2):
    from qlka import harness
    return harness.build_encoder(layers, kernel, dev, hidden=hidden, heads=heads, intermediate=2 * hidden, seed=3)


@pytest.mark.parametrize("kernel", KERNELS)
def test_nomic_padding_is_the_key_mask(dev, kernel):
    model = _nomic(dev, kernel)
    torch.manual_seed(4)
    L, S = 300, 420
    ids = torch.randint(1, 1000, (1, L), device=dev)
    padded = torch.zeros(2, S, dtype=torch.long, device=dev)
    padded[0, :L] = ids[0]
    padded[1] = torch.randint(1, 1000, (S,), device=dev)          # a second, unpadded document in the batch
    mask = torch.ones(2, S, dtype=torch.long, device=dev)
    mask[0, L:] = 0
    with torch.no_grad():
        alone = model(input_ids=ids, attention_mask=torch.ones_like(ids)).last_hidden_state
        batch = model(input_ids=padded, attention_mask=mask).last_hidden_state
    np.testing.assert_allclose(batch[0, :L].cpu().numpy(), alone[0].cpu().numpy(), rtol=2e-4, atol=2e-4,
                               err_msg=f"{kernel}: padded keys leak into real tokens")


@pytest.mark.parametrize("kernel", KERNELS)
def test_nomic_layer_attention_vs_float64(dev, kernel):
    from transformers.models.nomic_bert.modeling_nomic_bert import apply_rotary_pos_emb
    model = _nomic(dev, kernel, layers=1)
    attn = model.layers[0].self_attn
    captured = {}

    def hook(mod, args, kwargs, out):
        captured.update(kwargs)
        captured["hidden"] = args[0] if args else kwargs["hidden_states"]
        captured["out"] = out[0]

    h = attn.register_forward_hook(hook, with_kwargs=True)
    ids = torch.randint(1, 1000, (2, 200), device=dev)
    mask = torch.ones(2, 200, dtype=torch.long, device=dev)
    mask[0, 130:] = 0
    with torch.no_grad():
        model(input_ids=ids, attention_mask=mask)
    h.remove()
    x, (cos, sin) = captured["hidden"], captured["position_embeddings"]
    B, S, _ = x.shape
    shape = (B, S, -1, attn.head_dim)
    with torch.no_grad():
        q = attn.q_proj(x).view(shape).transpose(1, 2)
        k = attn.k_proj(x).view(shape).transpose(1, 2)
        v = attn.v_proj(x).view(shape).transpose(1, 2)
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        att = _dense_attention(kernel, q, k, v, attn.tau, mask.bool())
        want = torch.nn.functional.linear(att.transpose(1, 2).reshape(B, S, -1), attn.o_proj.weight.cpu().double())
    np.testing.assert_allclose(captured["out"].cpu().double().numpy(), want.numpy(), rtol=1e-4, atol=1e-5)


def test_harness_runs(dev):
    from qlka import harness
    r = harness.run("add_riesz", seq_len=256, batch_size=2, docs=3, layers=1, device=str(dev), hidden=128, heads=2,
                    intermediate=256)
    assert r["ms_per_doc"] > 0 and r["num_docs"] == 3
