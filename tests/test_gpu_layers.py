"""GPU parity of the fused attention layers (qlka.layers, qlka_layer_fwd) for add_laplace, add_riesz and add_bump.

* Against the same ops with the reference's torch epilogue (oracle/dense.py's add_*_layer, attention.py:67-92): the
  fused call must reproduce them to fp32 rounding of the epilogue.
* Against the float64 normalised kernel matrix (kernels.py:68-89 restated in oracle/dense.py), with and without a
  key mask (attention.py:119-124), at sizes where the matrix is cheap.
* The gradient path of add_riesz / add_bump (the reference's formulas over the differentiable op) and the
  forward-only add_laplace.
* The in-kernel key mask (qlka_layer_fwd_masked): against the reference's composition over zeroed keys with the
  n_pad corrections, evaluated in float64 (attention.py:122-124); bit-equal to the unmasked layer when nothing is
  masked; exactly zero rows for a p whose keys are all masked.
"""
import numpy as np
import pytest
import torch

from oracle import dense

pytestmark = pytest.mark.gpu

KERNELS = ("add_laplace", "add_riesz", "add_bump")
SHAPES = [  # P, D, N, M, C
    (2, 3, 40, 40, 8),
    (3, 5, 257, 190, 5),        # M != N, odd C
    (2, 4, 1000, 1000, 64),
    (1, 2, 300, 300, 128),      # two channel slots per lane
]


def _inputs(P, D, N, M, C, seed, dev, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(P, D, M, generator=g) * scale).to(dev)
    k = (torch.randn(P, D, N, generator=g) * scale).to(dev)
    v = torch.randn(P, N, C, generator=g).to(dev)
    return q, k, v


def _ops():
    from weighted_abs_sum import weighted_abs_sum_full
    from weighted_laplace_sum import weighted_laplace_sum
    return weighted_abs_sum_full, weighted_laplace_sum


def _op_layer(kernel, q, k, v, n_pad):
    abs_full, lap = _ops()
    if kernel == "add_laplace":
        return dense.add_laplace_layer(q, k, v, n_pad, lap)
    if kernel == "add_riesz":
        return dense.add_riesz_layer(q, k, v, n_pad, abs_full)
    return dense.add_bump_layer(q, k, v, n_pad, abs_full)


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("shape", SHAPES)
def test_fused_layer_matches_op_layer(dev, kernel, shape):
    from qlka import layers
    P, D, N, M, C = shape
    q, k, v = _inputs(P, D, N, M, C, seed=sum(shape), dev=dev, scale=0.7)
    for n_pad in (0, torch.arange(P, device=dev, dtype=torch.float32).reshape(P, 1) * 0.25):
        got = layers.layer_forward(kernel, q, k, v, n_pad)
        want = _op_layer(kernel, q, k, v, n_pad)
        assert got.shape == (P, M, C)
        np.testing.assert_allclose(got.cpu().numpy(), want.cpu().numpy(), rtol=2e-5, atol=2e-6,
                                   err_msg=f"{kernel} {shape} n_pad={n_pad if isinstance(n_pad, int) else 'per-p'}")


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("masked", [False, True])
def test_attention_vs_float64_kernel_matrix(dev, kernel, masked):
    from qlka import layers
    B, H, S, Dh = 2, 3, 200, 16
    g = torch.Generator().manual_seed(11)
    qa, ka, va = (torch.randn(B, H, S, Dh, generator=g) for _ in range(3))
    keep = None
    if masked:
        keep = torch.ones(B, S, dtype=torch.bool)
        keep[0, 150:] = False
        keep[1, 37:60] = False
    tau = dense.TAU[kernel]
    out = layers.attention(qa.to(dev), ka.to(dev), va.to(dev), kernel, tau,
                           None if keep is None else keep.to(dev)).cpu()
    q64 = qa.double().transpose(2, 3).reshape(B * H, Dh, S)
    k64 = ka.double().transpose(2, 3).reshape(B * H, Dh, S)
    v64 = va.double().reshape(B * H, S, Dh)
    mask = None if keep is None else keep.repeat_interleave(H, dim=0).double()
    A = dense.dense_kernel_matrix(kernel, q64, k64, tau, mask)
    ref = (A @ v64) / A.sum(dim=2, keepdim=True).clamp_min(dense.CLAMP)
    np.testing.assert_allclose(out.reshape(B * H, S, Dh).numpy(), ref.numpy(), rtol=2e-4, atol=2e-5,
                               err_msg=f"{kernel} masked={masked}")


@pytest.mark.parametrize("kernel", ("add_riesz", "add_bump"))
def test_layer_gradient_path(dev, kernel):
    from qlka import layers
    P, D, N, M, C = 2, 3, 60, 60, 4
    q, k, v = _inputs(P, D, N, M, C, seed=5, dev=dev, scale=0.8)
    fused = layers.LAYERS[kernel](q, k, v, 0)
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = layers.LAYERS[kernel](qg, kg, vg, 0)
    np.testing.assert_allclose(out.detach().cpu().numpy(), fused.cpu().numpy(), rtol=2e-5, atol=2e-6)
    wgt = torch.randn(out.shape, generator=torch.Generator().manual_seed(9)).to(dev)
    (out * wgt).sum().backward()
    # float64 reference through autograd of the dense layer
    q64, k64, v64 = (t.detach().cpu().double().requires_grad_(True) for t in (q, k, v))
    A = dense.dense_kernel_matrix(kernel, q64, k64)
    ref = (A @ v64) / A.sum(dim=2, keepdim=True).clamp_min(dense.CLAMP)
    (ref * wgt.cpu().double()).sum().backward()
    for name, got, want in (("q", qg.grad, q64.grad), ("k", kg.grad, k64.grad), ("v", vg.grad, v64.grad)):
        scale = want.abs().max().item()
        np.testing.assert_allclose(got.cpu().numpy(), want.numpy(), rtol=1e-3, atol=1e-4 * scale,
                                   err_msg=f"{kernel} grad_{name}")


def test_add_laplace_is_forward_only(dev):
    from qlka import layers
    q, k, v = _inputs(1, 2, 16, 16, 4, seed=1, dev=dev)
    with pytest.raises(RuntimeError, match="no backward"):
        layers.add_laplace(q.requires_grad_(True), k, v)
    with torch.no_grad():
        assert layers.add_laplace(q, k, v).shape == (1, 16, 4)


def test_layer_validation(dev):
    from qlka import layers
    q, k, v = _inputs(1, 2, 16, 16, 4, seed=1, dev=dev)
    with pytest.raises(ValueError):
        layers.layer_forward("softmax", q, k, v)
    with pytest.raises(RuntimeError, match="float32"):
        layers.layer_forward("add_riesz", q.double(), k, v)
    with pytest.raises(RuntimeError, match="CUDA"):
        layers.layer_forward("add_riesz", q.cpu(), k, v)


MASK_SHAPES = [  # P, D, N, M, C
    (3, 3, 40, 40, 8),
    (3, 4, 300, 400, 5),        # M != N, odd C, partial last key range. M >= N: add_riesz's den counts keys as
                                # S = M (attention.py:78), so for M < N - n_pad it is a difference of large terms
    (3, 4, 1000, 1000, 64),
    (2, 2, 300, 300, 128),      # two channel slots per lane
]


def _mask(P, N, seed, dev):
    g = torch.Generator().manual_seed(seed)
    keep = torch.rand(P, N, generator=g) < 0.7
    keep[0, N // 3: N // 3 + min(N // 2, 150)] = False     # a masked run over whole key ranges
    if P > 2:
        keep[2] = False                                    # every key masked
    return keep.to(dev)


def _reference_masked(kernel, q, k, v, keep):
    """attention.py:122-124 then attention.py:67-92, in float64 on the CPU with dense ops (kernels.py:73,81)."""
    q64, k64, v64 = (t.detach().cpu().double() for t in (q, k, v))
    kp = keep.cpu().double()
    k64, v64 = k64 * kp[:, None, :], v64 * kp[:, :, None]
    n_pad = k.shape[2] - kp.sum(dim=1, keepdim=True)

    def abs_full(a, b, c):
        return dense.dense_abs_sum(a, b, c)

    def lap(a, b, c):
        return dense.dense_laplace_sum(a, b, c)

    if kernel == "add_laplace":
        return dense.add_laplace_layer(q64, k64, v64, n_pad, lap)
    if kernel == "add_riesz":
        return dense.add_riesz_layer(q64, k64, v64, n_pad, abs_full)
    return dense.add_bump_layer(q64, k64, v64, n_pad, abs_full)


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("shape", MASK_SHAPES)
def test_masked_layer_matches_reference_composition(dev, kernel, shape):
    from qlka import layers
    P, D, N, M, C = shape
    print(f"masked {kernel} {shape}", flush=True)
    q, k, v = _inputs(P, D, N, M, C, seed=sum(shape) + 3, dev=dev, scale=0.7)
    keep = _mask(P, N, seed=sum(shape), dev=dev)
    got = layers.layer_forward(kernel, q, k, v, keep=keep).cpu().double()
    want = _reference_masked(kernel, q, k, v, keep)
    assert got.shape == (P, M, C)
    np.testing.assert_allclose(got.numpy(), want.numpy(), rtol=1e-4, atol=1e-5, err_msg=f"{kernel} {shape}")
    if P > 2:
        assert torch.all(got[2] == 0), "a p with every key masked gives zero rows"


@pytest.mark.parametrize("kernel", ("add_riesz", "add_bump"))
@pytest.mark.parametrize("kept,far", [(2, True), (3, True), (40, True), (40, False)])
def test_masked_layer_few_kept_keys_among_far_masked_keys(dev, kernel, kept, far):
    """A short document padded to a long length: p = 0 keeps 2, 3 or 40 of 4200 keys. With `far` the masked keys lie
    far above and below the kept ones (+-60 .. 80 against keys of scale 0.7), so that the largest and smallest keys of
    the segment are masked; otherwise they keep their values, interleaved with the kept ones. The masked abs walk must
    measure its distances and segment totals between kept keys (fill_masked_keys), and add_riesz's masked denominator
    must not cancel (S - n_pad formed exactly), to meet the masked-layer bar; p = 1 is an ordinary mask.
    Self-attention shape (M = N): add_riesz's denominator counts the sequence as S = M keys (attention.py:78) and
    clamps when M falls below the padded count."""
    from qlka import layers
    P, D, N, M, C = 2, 4, 4200, 4200, 16
    q, k, v = _inputs(P, D, N, M, C, seed=40 + kept, dev=dev, scale=0.7)
    keep = _mask(P, N, seed=41, dev=dev)
    keep[0] = False
    sel = [17, 2101, 4003][:kept] if kept <= 3 else list(range(5, N, N // kept))[:kept]
    keep[0, torch.tensor(sel, device=dev)] = True
    if far:
        dist = torch.linspace(60.0, 80.0, N, device=dev)
        side = torch.where(torch.arange(N, device=dev) % 2 == 0, 1.0, -1.0)
        k[0] = torch.where(keep[0][None, :], k[0], (side * dist)[None, :])
    got = layers.layer_forward(kernel, q, k, v, keep=keep).cpu().double()
    want = _reference_masked(kernel, q, k, v, keep)
    np.testing.assert_allclose(got.numpy(), want.numpy(), rtol=1e-4, atol=1e-5,
                               err_msg=f"{kernel} kept={kept} far={far}")


@pytest.mark.parametrize("kernel", KERNELS)
def test_masked_layer_without_masked_keys_is_the_unmasked_layer(dev, kernel):
    from qlka import layers
    P, D, N, M, C = 2, 3, 500, 400, 16
    q, k, v = _inputs(P, D, N, M, C, seed=77, dev=dev, scale=0.7)
    keep = torch.ones(P, N, dtype=torch.bool, device=dev)
    got = layers.layer_forward(kernel, q, k, v, keep=keep)
    want = layers.layer_forward(kernel, q, k, v)
    assert torch.equal(got, want)


@pytest.mark.parametrize("kernel", KERNELS)
def test_masked_layer_vs_reference_route_on_gpu(dev, kernel):
    # the reference's own GPU route (zeroed keys through the ops, n_pad epilogue) agrees with the in-kernel mask
    from qlka import layers
    P, D, N, M, C = 3, 4, 700, 700, 32
    q, k, v = _inputs(P, D, N, M, C, seed=5, dev=dev, scale=0.7)
    keep = _mask(P, N, seed=6, dev=dev)
    keep[2, :5] = True                                     # keep the all-masked p off this comparison's den clamp
    kf = keep.float()
    n_pad = N - kf.sum(dim=1, keepdim=True)
    route = layers.layer_forward(kernel, q, k * kf[:, None, :], v * kf[:, :, None], n_pad)
    got = layers.layer_forward(kernel, q, k, v, keep=keep)
    want = _reference_masked(kernel, q, k, v, keep)
    np.testing.assert_allclose(got.cpu().double().numpy(), want.numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(route.cpu().double().numpy(), want.numpy(), rtol=1e-3, atol=1e-4)


def test_masked_layer_validation(dev):
    from qlka import layers
    q, k, v = _inputs(2, 2, 16, 16, 4, seed=1, dev=dev)
    with pytest.raises(RuntimeError, match="keep must be"):
        layers.layer_forward("add_riesz", q, k, v, keep=torch.ones(2, 15, dtype=torch.bool, device=dev))


# Seeded random shapes, including ill-conditioned ones (wide spreads, a handful of keys or queries, add_riesz whose
# denominator cancels, add_bump queries with no key within distance 1): there the output is rounding noise of the
# epilogue's cancellation for any fp32 evaluation, the reference's own included, so no fixed tolerance between two fp32
# evaluations holds. The bar is relative to the reference: against the float64 evaluation of the same composition,
# the fused layer's largest error is at most twice that of the reference's fp32 composition (the ops + torch epilogue,
# over zeroed keys with n_pad for a mask), plus 1e-5 of the output scale.
def _random_layer_cases(n=16, seed=5):
    rng = np.random.default_rng(np.random.PCG64(seed))
    widths = (1, 2, 3, 5, 8, 16, 31, 32, 33, 63, 64, 65, 100, 127, 128)
    out = []
    while len(out) < n:
        P, D = int(rng.integers(1, 6)), int(rng.integers(1, 17))
        N = int(np.clip(np.exp(rng.uniform(0, np.log(3000))), 1, 3000))
        M = N if rng.random() < 0.5 else int(np.clip(np.exp(rng.uniform(0, np.log(3000))), 1, 3000))
        C = int(rng.choice(widths))
        if P * D * N * M > 3e7:
            continue
        out.append((P, D, N, M, C, str(rng.choice(KERNELS)), float(rng.choice([0.3, 0.7, 2.0])),
                    bool(rng.random() < 0.4), int(rng.integers(0, 1 << 20))))
    return out


# plus shapes a wider sweep of the same generator found where the two fp32 evaluations differ by up to 1e-3 relative
# (denominators that cancel) or, for add_bump with one key, by O(1) on rows that are 0 / 0 in exact arithmetic
RANDOM_LAYER_CASES = _random_layer_cases() + [
    (2, 14, 494, 77, 8, "add_riesz", 0.3, False, 551394),
    (1, 1, 2980, 6, 8, "add_riesz", 2.0, False, 276024),
    (5, 2, 1, 4, 128, "add_bump", 2.0, False, 424025),
    (2, 2, 16, 20, 2, "add_bump", 2.0, False, 936295),
]


@pytest.mark.parametrize("case", RANDOM_LAYER_CASES,
                         ids=[f"{c[5]}-P{c[0]}D{c[1]}N{c[2]}M{c[3]}C{c[4]}-s{c[6]}{'-masked' if c[7] else ''}"
                              for c in RANDOM_LAYER_CASES])
def test_random_layer_shapes_vs_float64(dev, case):
    from qlka import layers
    P, D, N, M, C, kernel, scale, masked, seed = case
    print(f"random layer {case}", flush=True)
    q, k, v = _inputs(P, D, N, M, C, seed=seed, dev=dev, scale=scale)
    if masked:
        keep = _mask(P, N, seed=seed, dev=dev)
        got = layers.layer_forward(kernel, q, k, v, keep=keep).cpu().double()
        kp = keep.float()
        n_pad = N - kp.sum(dim=1, keepdim=True)
        op = _op_layer(kernel, q, k * kp[:, None, :], v * kp[:, :, None], n_pad).cpu().double()
        ref = _reference_masked(kernel, q, k, v, keep)
    else:
        n_pad = torch.arange(P, device=dev, dtype=torch.float32).reshape(P, 1) * 0.25
        got = layers.layer_forward(kernel, q, k, v, n_pad).cpu().double()
        op = _op_layer(kernel, q, k, v, n_pad).cpu().double()
        q64, k64, v64 = (t.cpu().double() for t in (q, k, v))
        lap, absf = dense.dense_laplace_sum, dense.dense_abs_sum
        ref = (dense.add_laplace_layer(q64, k64, v64, n_pad.cpu().double(), lap) if kernel == "add_laplace" else
               dense.add_riesz_layer(q64, k64, v64, n_pad.cpu().double(), absf) if kernel == "add_riesz" else
               dense.add_bump_layer(q64, k64, v64, n_pad.cpu().double(), absf))
    assert got.shape == (P, M, C) and torch.all(torch.isfinite(got))
    e_fused = float((got - ref).abs().max())
    e_op = float((op - ref).abs().max())
    bar = 2.0 * e_op + 1e-5 * float(ref.abs().max()) + 1e-12
    assert e_fused <= bar, f"{case}: fused error {e_fused:.3e} > {bar:.3e} (reference composition's {e_op:.3e})"
