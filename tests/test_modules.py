"""Model-level integration (qlka.modules) on the CPU: parameter compatibility and plumbing.

With kernel="softmax" (scaled dot-product attention, scale tau**-2) the modules must reproduce the modules they
replace exactly: nn.MultiheadAttention for KernelMultiheadAttention (vision_transformer.py:19-44) and the HF
NomicBertAttention for KernelAttention (nomic.py:9-31), rotary embeddings and padding mask included. That pins the
projections, head split, mask extraction and output projection; the additive kernels through the same plumbing are
checked on the GPU (tests/test_gpu_modules.py).
"""

import pytest
import torch

from qlka import modules


def test_multihead_parameters_match_nn_multihead_attention():
    ref = torch.nn.MultiheadAttention(32, 4, batch_first=True)
    mod = modules.KernelMultiheadAttention(32, 4, kernel="add_riesz")
    want = {k: tuple(v.shape) for k, v in ref.state_dict().items()}
    got = {k: tuple(v.shape) for k, v in mod.state_dict().items()}
    assert got == want
    mod.load_state_dict(ref.state_dict())
    assert mod.tau == modules.TAU["add_riesz"]


def test_multihead_softmax_equals_nn_multihead_attention():
    torch.manual_seed(0)
    E, H = 32, 4
    ref = torch.nn.MultiheadAttention(E, H, batch_first=True)
    torch.nn.init.normal_(ref.in_proj_bias)
    mod = modules.KernelMultiheadAttention(E, H, kernel="softmax", tau=(E // H) ** 0.25)
    mod.load_state_dict(ref.state_dict())
    x = torch.randn(3, 11, E)
    want, _ = ref(x, x, x, need_weights=False)
    torch.testing.assert_close(mod(x), want, rtol=1e-5, atol=1e-6)


def _nomic(layers=2, hidden=64, heads=4):
    from transformers import NomicBertConfig, NomicBertModel
    torch.manual_seed(1)
    cfg = NomicBertConfig(num_hidden_layers=layers, hidden_size=hidden, num_attention_heads=heads,
                          intermediate_size=2 * hidden)
    return NomicBertModel._from_config(cfg, attn_implementation="sdpa").eval()


def test_nomic_kernel_attention_loads_and_matches_softmax():
    model = _nomic()
    ids = torch.randint(1, 1000, (2, 12))
    mask = torch.ones(2, 12, dtype=torch.long)
    mask[1, 7:] = 0
    with torch.no_grad():
        want = model(input_ids=ids, attention_mask=mask).last_hidden_state
        head_dim = model.config.hidden_size // model.config.num_attention_heads
        params = {n: p.data_ptr() for n, p in model.named_parameters()}
        modules.use_kernel_attention(model, "softmax", tau=head_dim ** 0.25)
        for layer in model.layers:
            assert layer.self_attn.qlka_kernel == ("softmax", head_dim ** 0.25, "efficient")
        assert model.config._attn_implementation == modules.REGISTRY_NAME
        assert {n: p.data_ptr() for n, p in model.named_parameters()} == params    # weights stay in place
        got = model(input_ids=ids, attention_mask=mask).last_hidden_state
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_nomic_standalone_kernel_attention_matches_layer():
    """KernelAttention(config, ...) takes a layer's state_dict and gives that layer's output under softmax."""
    model = _nomic(layers=1)
    head_dim = model.config.hidden_size // model.config.num_attention_heads
    layer = model.layers[0].self_attn
    attn = modules.KernelAttention(model.config, "softmax", tau=head_dim ** 0.25)
    attn.load_state_dict(layer.state_dict())
    assert model.config._attn_implementation == "sdpa"           # the model's own config is untouched
    x = torch.randn(2, 9, model.config.hidden_size)
    pos = model.rotary_emb(x, torch.arange(9)[None, :])
    with torch.no_grad():
        want, _ = layer(x, attention_mask=None, position_embeddings=pos)
        got, _ = attn(x, attention_mask=None, position_embeddings=pos)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_unsupported_kernels_and_impl():
    q = torch.randn(1, 2, 5, 4)
    with pytest.raises(NotImplementedError, match="does not run on the weighted"):
        modules.attention(q, q, q, "gauss", 1.0)
    with pytest.raises(NotImplementedError, match="naive"):
        modules.attention(q, q, q, "add_bump", 1.5, impl="naive")
    with pytest.raises(AssertionError):
        modules.attention(q, q, q, "add_bump", 1.5, impl="fast")


def test_harness_encoder_takes_its_sequence_length():
    # The encoder gathers its token-type buffer at the position ids (NomicBertEmbeddings), so a sequence longer than
    # max_position_embeddings indexes past that buffer: on the CPU torch raises, on the GPU the gather reads out of
    # bounds. The harness sizes the encoder to its seq_len.
    from qlka import harness
    S = 2100
    ids = torch.randint(1, 1000, (1, S))
    short = harness.build_encoder(1, "softmax", "cpu", hidden=32, heads=2, intermediate=64)
    with pytest.raises((IndexError, RuntimeError)):
        with torch.no_grad():
            short(input_ids=ids)
    model = harness.build_encoder(1, "softmax", "cpu", hidden=32, heads=2, intermediate=64, max_positions=S)
    assert model.config.max_position_embeddings == S
    with torch.no_grad():
        assert model(input_ids=ids).last_hidden_state.shape == (1, S, 32)
