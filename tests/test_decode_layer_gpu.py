"""The graph decoder's dense decode kernels (csrc/decode_layer.hip) against PyTorch.

References: torch.nn.functional.linear in float32 on the bf16 operands (then one bf16
rounding), transformers' Qwen3MoeRMSNorm module run in bf16 as the reference's
graphdec.py:160-181 runs it, the package's rope_decode kernel (bit-exact with the
oracle) and wisp.moe.route (graphdec.py:177). Sums run in another order than the
library kernels', so a bf16 result may sit one ulp away; the bars say so."""

import pytest
import torch
import torch.nn.functional as F

from wisp import kernels
from wisp.moe import route

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")
from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeRMSNorm  # noqa: E402

DEV = "cuda"


def _bf(*shape, std=1.0, gen=None):
    return (torch.randn(*shape, generator=gen, device=DEV) * std).to(torch.bfloat16)


def _ulps_off(got, ref):
    """Elementwise distance in units of the bf16 spacing at the reference value."""
    g, r = got.float(), ref.float()
    spacing = torch.clamp(r.abs(), min=1e-30)
    spacing = torch.pow(2.0, torch.floor(torch.log2(spacing)) - 7)
    return ((g - r).abs() / spacing)


def _linear_ref(W, x):
    return F.linear(x.float().view(1, -1), W.float()).view(-1).to(torch.bfloat16)


@pytest.mark.parametrize("O,K", [(5120, 2048), (2048, 4096), (128, 2048), (1000, 1024), (96, 256), (77, 520)])
def test_gemv_matches_linear(O, K):
    g = torch.Generator(device=DEV).manual_seed(O + K)
    W, x = _bf(O, K, std=0.02, gen=g), _bf(K, gen=g)
    y = torch.empty(O, dtype=torch.bfloat16, device=DEV)
    kernels.dl_gemv(y, W, x)
    torch.cuda.synchronize()
    off = _ulps_off(y, _linear_ref(W, x))
    print(f"gemv O={O} K={K}: max {off.max().item():.2f} ulp, {(off > 0).float().mean().item():.4f} differ")
    assert off.max().item() <= 1.0
    assert (off > 0).float().mean().item() < 0.05


def test_gemv_row_blocks_and_residual():
    g = torch.Generator(device=DEV).manual_seed(7)
    K = 2048
    Wq, Wk, Wv = _bf(4096, K, std=0.02, gen=g), _bf(512, K, std=0.02, gen=g), _bf(512, K, std=0.02, gen=g)
    x, res = _bf(K, gen=g), _bf(5120, gen=g)
    y = torch.empty(5120, dtype=torch.bfloat16, device=DEV)
    kernels.dl_gemv(y, Wq, x, w1=Wk, w2=Wv)
    ref = _linear_ref(torch.cat([Wq, Wk, Wv]), x)
    assert _ulps_off(y, ref).max().item() <= 1.0
    kernels.dl_gemv(y, Wq, x, w1=Wk, w2=Wv, res=res)
    ref2 = (res.float() + ref.float()).to(torch.bfloat16)  # the residual add in bf16, as h + o_proj(o)
    torch.cuda.synchronize()
    assert _ulps_off(y, ref2).max().item() <= 1.0


@pytest.mark.parametrize("K,with_b", [(2048, True), (2048, False), (256, True), (4096, False)])
def test_gemv_norm_prologue_matches_rmsnorm_module(K, with_b):
    g = torch.Generator(device=DEV).manual_seed(K + with_b)
    O = 128
    a, b = _bf(K, gen=g), _bf(K, gen=g)
    W = _bf(O, K, std=0.05, gen=g)
    norm = Qwen3MoeRMSNorm(K, eps=1e-6).to(DEV, torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(1.0 + 0.1 * torch.randn(K, generator=g, device=DEV))
    h_ref = (a.float() + b.float()).to(torch.bfloat16) if with_b else a
    x_ref = norm(h_ref.view(1, K)).view(K)
    y = torch.empty(O, dtype=torch.bfloat16, device=DEV)
    h_out = torch.empty(K, dtype=torch.bfloat16, device=DEV)
    x_out = torch.empty(K, dtype=torch.bfloat16, device=DEV)
    kernels.dl_gemv(y, W, a, b=b if with_b else None, norm_w=norm.weight.data, eps=1e-6, h_out=h_out, x_out=x_out)
    torch.cuda.synchronize()
    assert torch.equal(h_out.view(torch.int16), h_ref.view(torch.int16))
    offx = _ulps_off(x_out, x_ref)
    print(f"rmsnorm K={K}: max {offx.max().item():.2f} ulp, {(offx > 0).float().mean().item():.4f} differ")
    assert offx.max().item() <= 1.0 and (offx > 0).float().mean().item() < 0.02
    # y is W applied to the kernel's own x
    assert _ulps_off(y, _linear_ref(W, x_out)).max().item() <= 1.0


def test_gemv_embedding_row():
    g = torch.Generator(device=DEV).manual_seed(3)
    V, K, O = 500, 1024, 64
    emb, W = _bf(V, K, gen=g), _bf(O, K, std=0.05, gen=g)
    nw = torch.ones(K, dtype=torch.bfloat16, device=DEV)
    tok = torch.tensor([321], dtype=torch.int64, device=DEV)
    h_out = torch.empty(K, dtype=torch.bfloat16, device=DEV)
    y = torch.empty(O, dtype=torch.bfloat16, device=DEV)
    kernels.dl_gemv(y, W, emb, a_row=tok, norm_w=nw, eps=1e-6, h_out=h_out)
    torch.cuda.synchronize()
    assert torch.equal(h_out, emb[321])


@pytest.mark.parametrize("Hq,Hk,D", [(32, 4, 128), (4, 2, 64), (8, 8, 256)])
def test_qk_rope_matches_modules(Hq, Hk, D):
    g = torch.Generator(device=DEV).manual_seed(Hq * D)
    tmax, pos = 96, 37
    qkv = _bf((Hq + 2 * Hk) * D, gen=g)
    qn = Qwen3MoeRMSNorm(D, eps=1e-6).to(DEV, torch.bfloat16)
    kn = Qwen3MoeRMSNorm(D, eps=1e-6).to(DEV, torch.bfloat16)
    with torch.no_grad():
        qn.weight.copy_(1.0 + 0.2 * torch.randn(D, generator=g, device=DEV))
        kn.weight.copy_(1.0 + 0.2 * torch.randn(D, generator=g, device=DEV))
    ang = torch.arange(tmax, device=DEV)[:, None] * (1.0 / 1e4 ** (torch.arange(0, D, 2, device=DEV) / D))[None]
    ang = torch.cat([ang, ang], 1)
    cos, sin = ang.cos().to(torch.bfloat16).contiguous(), ang.sin().to(torch.bfloat16).contiguous()
    kc = torch.zeros(1, Hk, tmax, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    qo = torch.empty(Hq * D, dtype=torch.bfloat16, device=DEV)
    p = torch.tensor([pos], dtype=torch.int64, device=DEV)
    kernels.dl_qk_rope(qkv, qn.weight.data, kn.weight.data, 1e-6, cos, sin, p, Hq, Hk, D, kc, vc, qo)
    # the modules' path: q_norm / k_norm, then rope_decode, then index_copy_ at pos
    q = qn(qkv[: Hq * D].view(1, 1, Hq, D)).transpose(1, 2)
    k = kn(qkv[Hq * D : (Hq + Hk) * D].view(1, 1, Hk, D)).transpose(1, 2)
    q, k = kernels.rope_decode(q, k, cos[pos].view(1, 1, D), sin[pos].view(1, 1, D))
    torch.cuda.synchronize()
    offq = _ulps_off(qo.view(Hq, D), q.reshape(Hq, D))
    offk = _ulps_off(kc[0, :, pos], k.reshape(Hk, D))
    print(f"qk_rope Hq={Hq} D={D}: q max {offq.max().item():.2f} ulp ({(offq > 0).float().mean().item():.4f}), "
          f"k max {offk.max().item():.2f} ulp")
    # a one-ulp difference of a normed element moves the rotated value by up to ~2 ulp
    assert offq.max().item() <= 2.0 and (offq > 0).float().mean().item() < 0.05
    assert offk.max().item() <= 2.0 and (offk > 0).float().mean().item() < 0.05
    assert torch.equal(vc[0, :, pos].reshape(-1), qkv[(Hq + Hk) * D :])
    others = torch.ones(tmax, dtype=torch.bool, device=DEV)
    others[pos] = False
    assert kc[0][:, others].abs().sum().item() == 0 and vc[0][:, others].abs().sum().item() == 0


@pytest.mark.parametrize("Hq,Hk,D,T", [(32, 4, 128, 4096), (32, 4, 128, 300), (8, 8, 64, 130), (4, 1, 256, 70),
                                       (32, 2, 128, 64), (16, 4, 128, 200), (4, 2, 64, 65)])
def test_qk_rope_attn_equals_the_two_calls(Hq, Hk, D, T):
    """The fused launch pair (q/k head norm + rope + K/V store inside the attention
    workgroups) against dl_qk_rope then attn_decode: the output, the K and V written at pos
    and every other cache row equal bit for bit, at chunk edges and the last position."""
    g = torch.Generator(device=DEV).manual_seed(Hq * D + T)
    qn = (1.0 + 0.2 * torch.randn(D, generator=g, device=DEV)).to(torch.bfloat16)
    kn = (1.0 + 0.2 * torch.randn(D, generator=g, device=DEV)).to(torch.bfloat16)
    ang = torch.arange(T, device=DEV)[:, None] * (1.0 / 1e4 ** (torch.arange(0, D, 2, device=DEV) / D))[None]
    ang = torch.cat([ang, ang], 1)
    cos, sin = ang.cos().to(torch.bfloat16).contiguous(), ang.sin().to(torch.bfloat16).contiguous()
    kc0 = _bf(1, Hk, T, D, gen=g)
    vc0 = _bf(1, Hk, T, D, gen=g)
    scale = D ** -0.5
    for pos in sorted(p for p in {0, 1, 63, 64, 127, T // 2, T - 1} if p < T):
        qkv = _bf((Hq + 2 * Hk) * D, gen=g)
        p = torch.tensor([pos], dtype=torch.int64, device=DEV)
        ka, va = kc0.clone(), vc0.clone()
        qo = torch.empty(Hq * D, dtype=torch.bfloat16, device=DEV)
        kernels.dl_qk_rope(qkv, qn, kn, 1e-6, cos, sin, p, Hq, Hk, D, ka, va, qo)
        ref = kernels.attn_decode(qo.view(Hq, D), ka, va, p, scale)
        kb, vb = kc0.clone(), vc0.clone()
        got = kernels.dl_qk_rope_attn(qkv, qn, kn, 1e-6, cos, sin, p, Hq, Hk, D, kb, vb, scale)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), pos
        assert torch.equal(kb.view(torch.int16), ka.view(torch.int16)), pos
        assert torch.equal(vb.view(torch.int16), va.view(torch.int16)), pos


@pytest.mark.parametrize("E,k,norm", [(128, 8, True), (128, 8, False), (8, 2, True), (60, 4, True), (512, 10, True),
                                      (128, 16, True), (64, 1, True), (256, 8, True)])
def test_route_matches_moe_route(E, k, norm):
    g = torch.Generator(device=DEV).manual_seed(E * k)
    row = torch.empty(2 * k, dtype=torch.float32, device=DEV)
    checked = 0
    for _ in range(20):
        logits = (torch.randn(E, generator=g, device=DEV) * 2).to(torch.bfloat16)
        sel, rw = route(logits.view(1, E), k, norm, torch.bfloat16)
        p = torch.softmax(logits.float(), 0)
        top = torch.sort(p, descending=True).values
        if (top[k - 1] - top[k]).item() <= 1e-6 * top[k - 1].item():
            continue  # a tie at the boundary: either choice is the reference's
        kernels.dl_route(logits, k, norm, row)
        torch.cuda.synchronize()
        got_sel = row[:k].long()
        assert set(got_sel.tolist()) == set(sel[0].tolist())
        # same experts; compare the weight of each expert: bit for bit where the kernel sums
        # in torch's order (the softmax always; the renormalisation for k a power of two),
        # else within one bf16 ulp
        ref_w = {int(e): float(w) for e, w in zip(sel[0].tolist(), rw[0].float().tolist())}
        exact = not norm or (k & (k - 1)) == 0
        for e, w in zip(got_sel.tolist(), row[k:].tolist()):
            if exact:
                assert w == ref_w[e], (e, w, ref_w[e])
            else:
                assert abs(w - ref_w[e]) <= 2.0**-7 * abs(ref_w[e]) + 1e-12, (e, w, ref_w[e])
        # descending order, as torch.topk returns it
        assert all(row[k + i].item() >= row[k + i + 1].item() for i in range(k - 1))
        checked += 1
    assert checked >= 15


def test_route_signals_the_host_after_the_row():
    """With host buffers the route kernel also writes the row to pinned host memory and then
    bumps the host flag (graphdec.py:305's per-layer sync without a stream sync)."""
    g = torch.Generator(device=DEV).manual_seed(5)
    E, k = 128, 8
    row = torch.empty(2 * k, dtype=torch.float32, device=DEV)
    host_row = torch.zeros(3 * k, dtype=torch.float32, pin_memory=True)
    flag = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    seq = torch.zeros(1, dtype=torch.int32, device=DEV)
    for it in range(4):
        logits = torch.randn(E, generator=g, device=DEV).to(torch.bfloat16)
        kernels.dl_route(logits, k, True, row, host_row, flag, seq)
        torch.cuda.synchronize()
        assert int(flag[0]) == it + 1 and int(seq.item()) == it + 1
        assert torch.equal(host_row[: 2 * k], row.cpu())
