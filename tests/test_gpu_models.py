"""GPU tests of the callers of the path: ViT-T / Swin-T with the ELSA drop-ins against the
same models on PyTorch SDPA (forward and gradients), the reference's toy-encoder pair
test (tests/test_attention.py:116-130), and a hipGraph capture of the patched forward
replayed several times with eager work in between."""
from __future__ import annotations

import copy

import pytest
import torch

import elsa_amd
from elsa_amd.vision_models import SwinTransformer, swin_tiny_patch4_window7, vit_tiny_patch16
from tests.gpu_util import describe

pytestmark = pytest.mark.gpu


def swin_tiny_window_ratio8(img_size: int) -> SwinTransformer:
    """Swin-T at the reference benchmark's geometry: window = (img/4) / window_ratio with
    window_ratio 8 (benchmarks/bench_timm_dropin.py:38-49, :60), so 12x12 windows (144 tokens)
    at 384 px and 16x16 (256 tokens) at 512 px, shifted, with the relative-position bias."""
    return SwinTransformer(img_size=img_size, embed_dim=96, depths=(2, 2, 6, 2), num_heads=(3, 6, 12, 24),
                           window_size=img_size // 4 // 8)


def _models(builder, img, dtype, train=False):
    torch.manual_seed(1234)
    base = builder(img).eval()
    elsa = copy.deepcopy(base)
    (elsa_amd.patch_timm_attention_train if train else elsa_amd.patch_timm_attention)(elsa)
    ref32 = copy.deepcopy(base).to("cuda", torch.float32)
    return ref32, elsa.to("cuda", dtype)


@pytest.mark.parametrize("dt,tol", [(torch.float32, 2e-4), (torch.float16, 2e-2)])
@pytest.mark.parametrize("builder,img,batch", [(vit_tiny_patch16, 224, 2), (swin_tiny_patch4_window7, 224, 2),
                                               (vit_tiny_patch16, 512, 2), (vit_tiny_patch16, 1024, 8),
                                               (vit_tiny_patch16, 2048, 2),  # 16385 tokens: B2 H3 N16385
                                               (swin_tiny_patch4_window7, 384, 8),
                                               (swin_tiny_patch4_window7, 512, 8),
                                               (swin_tiny_window_ratio8, 384, 4),
                                               (swin_tiny_window_ratio8, 512, 4)])
def test_dropin_forward_matches_sdpa(builder, img, batch, dt, tol):
    describe(f"dropin fwd {builder.__name__} {img} batch {batch} {dt}")
    ref, elsa = _models(builder, img, dt)
    x = torch.randn(batch, 3, img, img, generator=torch.Generator().manual_seed(7)).cuda()
    with torch.no_grad():
        want = ref(x)
        got = elsa(x.to(dt)).float()
    err = (got - want).abs().max().item()
    describe(f"  max_abs logits {err:.3e}")
    assert err <= tol * max(1.0, want.abs().max().item())


# the training step above 224 px at the reference's published training sizes (README.md:73-76:
# ViT 384/512/768, Swin 384/512) and BASELINE's ViT 1024 / 2048 px rows
TRAIN_FP32 = [(vit_tiny_patch16, 224, 2), (swin_tiny_patch4_window7, 224, 2), (vit_tiny_patch16, 512, 2),
              (vit_tiny_patch16, 1024, 2), (vit_tiny_patch16, 2048, 1), (swin_tiny_patch4_window7, 384, 2),
              (swin_tiny_patch4_window7, 512, 2), (swin_tiny_window_ratio8, 384, 2),
              (swin_tiny_window_ratio8, 512, 2)]


@pytest.mark.parametrize("builder,img,batch", TRAIN_FP32,
                         ids=[f"{b.__name__}-{i}-b{n}" for b, i, n in TRAIN_FP32])
def test_dropin_training_gradients_match_sdpa(builder, img, batch):
    describe(f"dropin train {builder.__name__} {img} batch {batch}")
    ref, elsa = _models(builder, img, torch.float32, train=True)
    ref.train()
    elsa.train()
    g = torch.Generator().manual_seed(11)
    x = torch.randn(batch, 3, img, img, generator=g).cuda()
    labels = torch.randint(0, 1000, (batch,), generator=g).cuda()
    for m in (ref, elsa):
        torch.nn.functional.cross_entropy(m(x), labels).backward()
    worst = 0.0
    for (n, p), (_, q) in zip(ref.named_parameters(), elsa.named_parameters()):
        assert p.grad is not None and q.grad is not None, n
        err = (p.grad - q.grad).abs().max().item() / max(1e-6, p.grad.abs().max().item())
        worst = max(worst, err)
        assert err <= 2e-3, (n, err)
    describe(f"  worst relative grad error {worst:.3e}")


TRAIN_FP16 = [(vit_tiny_patch16, 224, 8), (swin_tiny_patch4_window7, 224, 8), (vit_tiny_patch16, 512, 8),
              (vit_tiny_patch16, 1024, 4), (vit_tiny_patch16, 2048, 1), (swin_tiny_patch4_window7, 384, 8),
              (swin_tiny_patch4_window7, 512, 8), (swin_tiny_window_ratio8, 512, 4)]


@pytest.mark.parametrize("builder,img,batch", TRAIN_FP16,
                         ids=[f"{b.__name__}-{i}-b{n}" for b, i, n in TRAIN_FP16])
def test_dropin_fp16_training_is_as_accurate_as_sdpa_fp16(builder, img, batch):
    """fp16 training step: the gradients of the fp16 model with the ELSA drop-in and of the
    same fp16 model on SDPA, each against the fp32 SDPA model; ELSA's error may not exceed
    twice SDPA's (fp16 rounding everywhere else in the network sets both)."""
    describe(f"dropin fp16 train {builder.__name__} {img} batch {batch}")
    torch.manual_seed(1234)
    base = builder(img)
    elsa = copy.deepcopy(base)
    elsa_amd.patch_timm_attention_train(elsa)
    ref32 = copy.deepcopy(base).cuda().train()
    sdpa16 = copy.deepcopy(base).to("cuda", torch.float16).train()
    elsa16 = elsa.to("cuda", torch.float16).train()
    g = torch.Generator().manual_seed(12)
    x = torch.randn(batch, 3, img, img, generator=g).cuda()
    labels = torch.randint(0, 1000, (batch,), generator=g).cuda()
    for m, xx in ((ref32, x), (sdpa16, x.half()), (elsa16, x.half())):
        torch.nn.functional.cross_entropy(m(xx).float(), labels).backward()
    errs = {"sdpa16": 0.0, "elsa16": 0.0}
    for name, m in (("sdpa16", sdpa16), ("elsa16", elsa16)):
        for (n, p), (_, q) in zip(ref32.named_parameters(), m.named_parameters()):
            assert q.grad is not None and torch.isfinite(q.grad).all(), n
            rel = (p.grad - q.grad.float()).norm().item() / max(1e-12, p.grad.norm().item())
            errs[name] = max(errs[name], rel)
    describe(f"  worst relative grad error (norm) {errs}")
    assert errs["elsa16"] <= max(2.0 * errs["sdpa16"], 1e-2)


@pytest.mark.parametrize("dt,tol", [(torch.float32, 5e-3), (torch.float16, 8e-2)])
def test_full_model_pair_matches(dt, tol):
    torch.manual_seed(6)
    baseline, elsa = elsa_amd.make_model_pair(dim=96, depth=2, heads=3)
    baseline = baseline.eval().to(device="cuda", dtype=dt)
    elsa = elsa.eval().to(device="cuda", dtype=dt)
    x = torch.randn((1, 128, 96), device="cuda", dtype=dt)
    with torch.no_grad():
        torch.testing.assert_close(elsa(x), baseline(x), atol=tol, rtol=tol)


def test_train_model_pair_gradients():
    torch.manual_seed(7)
    base, elsa = elsa_amd.make_train_model_pair(dim=96, depth=2, heads=3, is_causal=True)
    base, elsa = base.cuda(), elsa.cuda()
    x = torch.randn((2, 200, 96), device="cuda")
    for m in (base, elsa):
        m(x).square().mean().backward()
    for (n, p), (_, q) in zip(base.named_parameters(), elsa.named_parameters()):
        torch.testing.assert_close(q.grad, p.grad, atol=5e-5, rtol=5e-3, msg=n)


def test_hipgraph_capture_of_patched_forward_replays():
    describe("hipgraph capture")
    _, elsa = _models(vit_tiny_patch16, 224, torch.float16)
    static_x = torch.randn(4, 3, 224, 224, device="cuda", dtype=torch.float16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), torch.no_grad():
        for _ in range(2):
            elsa(static_x)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph):
        static_y = elsa(static_x)
    for i in range(4):
        static_x.copy_(torch.randn_like(static_x))
        graph.replay()
        torch.cuda.synchronize()
        with torch.no_grad():
            eager = elsa(static_x)
        torch.cuda.synchronize()
        assert torch.equal(static_y, eager), i


@pytest.mark.parametrize("causal", [False, True])
def test_hipgraph_capture_of_forward_and_backward(causal):
    describe(f"hipgraph fwd+bwd causal={causal}")
    shape = (1, 3, 1031, 64)
    static = [torch.randn(shape, device="cuda", dtype=torch.float16) for _ in range(4)]
    q, k, v, do = static

    def run():
        out, rm, rz = elsa_amd.twopass_attention_with_state(q, k, v, is_causal=causal)
        return (out,) + tuple(elsa_amd.twopass_attention_backward(q, k, v, out, do, is_causal=causal, row_m=rm,
                                                                   row_z=rz))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run()
    g = torch.Generator(device="cuda").manual_seed(5)
    for i in range(3):
        for t in static:
            t.copy_(torch.randn(shape, device="cuda", dtype=torch.float16, generator=g))
        graph.replay()
        torch.cuda.synchronize()
        eager = run()
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "dq", "dk", "dv"), outs, eager):
            assert torch.equal(a, b), (i, name)
