"""Graph decoder on the GPU: a small Qwen3-MoE (transformers' own model class) whose experts
are 4-bit in the expert store, decoded with this package's kernels (rope_decode,
attn_decode, the MoE decode kernels) inside hipGraph segments, against the same model run
by transformers in float32 on the host with the dequantized expert weights. The pattern
follows the reference's tests/test_graphdec.py:49-129."""

import copy

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")
from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM  # noqa: E402

from wisp.cache import ExpertCache  # noqa: E402
from wisp.graphdec import GraphDecoder  # noqa: E402
from wisp.model import _fresh_rotary  # noqa: E402
from wisp.moe import Runtime, attach  # noqa: E402
from wisp.quant import dequant  # noqa: E402
from wisp.store import ExpertStore  # noqa: E402

H, I, E, K, L, G = 256, 128, 8, 2, 3, 128


def _models(seed=0, nslots=10, bits=4, fused=2):
    torch.manual_seed(seed)
    cfg = Qwen3MoeConfig(vocab_size=128, hidden_size=H, intermediate_size=256, moe_intermediate_size=I,
                         num_hidden_layers=L, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                         num_experts=E, num_experts_per_tok=K, norm_topk_prob=True, max_position_embeddings=512,
                         decoder_sparse_step=1, mlp_only_layers=[])
    ref = Qwen3MoeForCausalLM(cfg).eval()
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_(p.to(torch.bfloat16).float())  # weights the bf16 copy holds exactly
        store = ExpertStore(L, E, H * I, bits, G)
        for l, layer in enumerate(ref.model.layers):
            ex = layer.mlp.experts
            for e in range(E):
                w3 = torch.stack([ex.gate_up_proj[e, :I].reshape(-1), ex.gate_up_proj[e, I:].reshape(-1),
                                  ex.down_proj[e].reshape(-1)])
                store.put(l, e, w3, "cuda")
            W = dequant(store.host[l * E : (l + 1) * E].cuda(), H * I, bits, G).float().cpu()
            ex.gate_up_proj.copy_(torch.cat([W[:, 0].view(E, I, H), W[:, 1].view(E, I, H)], 1))
            ex.down_proj.copy_(W[:, 2].view(E, H, I))
    gpu = copy.deepcopy(ref).to("cuda", torch.bfloat16)
    _fresh_rotary(gpu, cfg, "cuda")
    rt = Runtime(store, fused=fused)
    rt.cache = ExpertCache(store, nslots)
    attach(gpu, rt)
    return cfg, ref, gpu, rt


def _close(got, ref, tol):
    g, r = got.float().cpu(), ref.float()
    err = ((g - r).norm() / r.norm()).item()
    return err, err <= tol


@pytest.mark.parametrize("use_graph", [True, False])
def test_decoder_matches_transformers(use_graph):
    cfg, ref, gpu, rt = _models()
    ids = torch.randint(0, 128, (1, 9), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        out = ref(input_ids=ids, use_cache=True)
        pk = out.past_key_values
        dec = GraphDecoder(gpu, rt, tmax=128, use_graph=use_graph)
        lg = dec.prefill(ids[0].cuda(), 0, chunk=4)
        err, ok = _close(lg, out.logits[:, -1], 2e-2)
        print(f"prefill rel-L2 {err:.3e}")
        assert ok, err
        t = out.logits[:, -1].argmax(-1)
        for step in range(6):
            r = ref(input_ids=t[:, None], past_key_values=pk, use_cache=True)
            pk = r.past_key_values
            got = dec.next(t.cuda())
            err, ok = _close(got, r.logits[:, -1], 2e-2)
            print(f"step {step} rel-L2 {err:.3e}")
            assert ok, (step, err)
            t = r.logits[:, -1].argmax(-1)
    st = rt.cache.core.stats
    assert st["misses"] > 0 and rt.stats["layer_calls"] >= 6 * L  # paging really happened
    rt.cache.free()


def test_graph_and_eager_decode_agree():
    cfg, ref, gpu, rt = _models(seed=3)
    ids = torch.randint(0, 128, (1, 5), generator=torch.Generator().manual_seed(4))
    outs = []
    for use_graph in (False, True):
        rt.cache.free()
        rt.cache = ExpertCache(rt.store, 10)
        dec = GraphDecoder(gpu, rt, tmax=64, use_graph=use_graph)
        with torch.no_grad():
            lg = dec.prefill(ids[0].cuda())
            seq = []
            t = lg.argmax(-1)
            for _ in range(5):
                lg = dec.next(t).clone()
                seq.append(lg)
                t = lg.argmax(-1)
        outs.append(torch.stack(seq))
    assert torch.allclose(outs[0].float(), outs[1].float(), rtol=1e-3, atol=1e-3)
    rt.cache.free()


@pytest.mark.parametrize("policy", ["lru", "wsa"])
def test_device_paging_with_partly_forced_routing_matches_host_steps(policy):
    """A decoder whose hook forces the experts of even layers only (None for the others: the
    router's choice): the graph with the paging points on the GPU gives the host-step
    decoder's logits bit for bit and the same cache state (slots, counters, free stack,
    ticks, scores, the frequency table and inc), under the LRU and the WSA policy."""
    cfg, ref, gpu, rt = _models(seed=5)
    ids = torch.randint(0, 128, (1, 4), generator=torch.Generator().manual_seed(6))
    rng = np.random.default_rng(7)
    draws = [[rng.choice(E, size=K, replace=False).astype(np.int64) for _ in range(L)] for _ in range(6)]

    class Half(GraphDecoder):
        def _expert_ids(self, i):
            return draws[self.pos - 4][i] if i % 2 == 0 else None

    outs, cores = [], []
    for paging in (False, True):
        rt.cache.free()
        rt.cache = ExpertCache(rt.store, 10, policy=policy)
        dec = Half(gpu, rt, tmax=64, device_paging=paging)
        with torch.no_grad():
            t = dec.prefill(ids[0].cuda()).argmax(-1)
            seq = []
            for _ in range(6):
                lg = dec.next(t).clone()
                seq.append(lg)
                t = lg.argmax(-1)
        assert dec._dev == paging and len(dec.graphs) == (1 if paging else L + 1)
        outs.append(torch.stack(seq))
        core = rt.cache.core
        cores.append((dict(core.key2slot), dict(core.stats), list(core.free), list(core.last), list(core.score),
                      list(core.freq.items()), core.inc))
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert cores[0] == cores[1]
    rt.cache.free()


class _DenseMoE(torch.nn.Module):
    """Dense reference MoE block with the attributes the decoder reads (gate, top_k,
    norm_topk, E, I, next_gate), as the reference's test stand-in (test_graphdec.py:12-35)."""

    def __init__(self, h, i, e, k):
        super().__init__()
        self.gate = torch.nn.Linear(h, e, bias=False)
        self.w1, self.w3, self.w2 = (torch.nn.Parameter(torch.randn(e, i, h) * 0.1),
                                     torch.nn.Parameter(torch.randn(e, i, h) * 0.1),
                                     torch.nn.Parameter(torch.randn(e, h, i) * 0.1))
        self.top_k, self.norm_topk, self.E, self.I, self.next_gate = k, True, e, i, None
        self.forced = None  # expert ids replacing the top-k of a one-token forward
        self.agreed = []  # per forced forward: were they this router's own top-k?

    def mix(self, x, sel, rw):
        y = torch.zeros_like(x)
        for e, w in zip(sel, rw, strict=True):
            y = y + w * (torch.nn.functional.silu(x @ self.w1[e].T) * (x @ self.w3[e].T)) @ self.w2[e].T
        return y

    def forward(self, h):
        x = h.reshape(-1, h.shape[-1])
        rw = torch.softmax(self.gate(x), dim=1, dtype=torch.float32)
        if self.forced is not None:
            sel = torch.tensor(self.forced).view(1, -1)
            self.agreed.append(set(self.forced) == set(torch.topk(rw, self.top_k, -1).indices[0].tolist()))
            rw = rw.gather(1, sel)
        else:
            rw, sel = torch.topk(rw, self.top_k, -1)
        rw = (rw / rw.sum(-1, keepdim=True)).to(x.dtype)
        return torch.stack([self.mix(x[t : t + 1], sel[t], rw[t])[0] for t in range(x.shape[0])]).view_as(h)


def test_prepare_and_moe_overrides_own_the_expert_step():
    """The reference's decoder test (test_graphdec.py:39-78): a subclass overrides the host
    step `_prepare(i, row)` (it receives the route row [expert ids | weights] of every layer)
    and `_moe(i)` (a dense MoE of those experts), with no runtime at all; decoding then
    matches transformers on the same model. Here the model is decoded in bf16 by this
    package's attention/router kernels against a float32 host run of the same bf16-exact
    weights (head_dim 64: the decode attention kernel takes head dims 64, 128 and 256).
    The host run takes each layer's experts from the row the decoder's _prepare received
    (its weights from its own router), so a near-tie that bf16 and float32 break apart
    cannot flip an expert between the two; nearly every choice must still be the host
    router's own top-k."""
    torch.manual_seed(0)
    cfg = Qwen3MoeConfig(vocab_size=100, hidden_size=64, intermediate_size=64, moe_intermediate_size=32,
                         num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                         num_experts=8, num_experts_per_tok=2, norm_topk_prob=True, max_position_embeddings=256,
                         decoder_sparse_step=1, mlp_only_layers=[])
    ref = Qwen3MoeForCausalLM(cfg).eval()
    for lay in ref.model.layers:
        lay.mlp = _DenseMoE(64, 32, 8, 2)
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_(p.to(torch.bfloat16).float())
    gpu = copy.deepcopy(ref).to("cuda", torch.bfloat16)
    _fresh_rotary(gpu, cfg, "cuda")
    rows = []

    class DenseDecoder(GraphDecoder):
        def _prepare(self, i, row):
            k = self.k
            rows.append((i, row))
            self.sel, self.w = [int(v) for v in row[:k]], row[k : 2 * k]

        def _moe(self, i):
            w = [torch.tensor(v, device=self.dev, dtype=self.dt) for v in self.w]
            return self.layers[i].mlp.mix(self.xn.view(1, -1), self.sel, w).view(1, 1, -1)

    ids = torch.randint(0, 100, (1, 7), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        out = ref(input_ids=ids, use_cache=True)
        pk, t = out.past_key_values, out.logits[:, -1].argmax(-1)
        dec = DenseDecoder(gpu, None, tmax=64, use_graph=False)
        dec.load_kv(pk, 7)
        for step in range(6):
            got = dec.next(t.cuda())
            for i, row in rows[-3:]:
                ref.model.layers[i].mlp.forced = [int(v) for v in row[:2]]
            r = ref(input_ids=t[:, None], past_key_values=pk, use_cache=True)
            for lay in ref.model.layers:
                lay.mlp.forced = None
            pk = r.past_key_values
            err, ok = _close(got, r.logits[:, -1], 2e-2)
            print(f"step {step} rel-L2 {err:.3e}")
            assert ok, (step, err)
            t = r.logits[:, -1].argmax(-1)
    assert not dec._dev and [i for i, _ in rows] == list(range(3)) * 6
    agreed = [a for lay in ref.model.layers for a in lay.mlp.agreed]
    assert len(agreed) == 18 and sum(agreed) >= 16, agreed  # the host router's own top-k (nearly) always
    for _, row in rows:  # [expert ids | normalised weights]
        assert len(row) == 4 and all(0 <= v < 8 and v == int(v) for v in row[:2]) and abs(sum(row[2:]) - 1) < 1e-2


def test_prefetch_and_recorder_paths_give_the_same_tokens():
    """The per-layer host step with prefetch of the next layer's predicted experts (and with a
    routing recorder) reads the row through the generic path; only slot placement may change,
    so the logits are bit-identical to the signalled fast path's."""
    cfg, ref, gpu, rt = _models(seed=7, nslots=12)
    ids = torch.randint(0, 128, (1, 6), generator=torch.Generator().manual_seed(8))
    outs = []
    for mode in ("fast", "prefetch", "recorder"):
        rt.cache.free()
        rt.cache = ExpertCache(rt.store, 12)
        rt.prefetch = mode == "prefetch"
        rt.recorder = [] if mode == "recorder" else None
        rt.reset_stats()
        dec = GraphDecoder(gpu, rt, tmax=64)
        with torch.no_grad():
            lg = dec.prefill(ids[0].cuda())
            seq, t = [], lg.argmax(-1)
            for _ in range(5):
                lg = dec.next(t).clone()
                seq.append(lg)
                t = lg.argmax(-1)
        outs.append(torch.stack(seq))
        if mode == "prefetch":
            assert rt.stats["prefetched"] > 0
        if mode == "recorder":
            assert len(rt.recorder) >= 5 * L
    rt.prefetch, rt.recorder = False, None
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    rt.cache.free()


def test_resize_and_reprefill_keep_context():
    cfg, ref, gpu, rt = _models(seed=5)
    ids = torch.randint(0, 128, (1, 20), generator=torch.Generator().manual_seed(6))
    with torch.no_grad():
        r = ref(input_ids=ids, use_cache=True)
        dec = GraphDecoder(gpu, rt, tmax=64)
        dec.prefill(ids[0, :12].cuda(), 0, chunk=5)
        lg = dec.prefill(ids[0, 12:].cuda(), 12, chunk=3)  # turn 2 reuses positions 0..11
        err, ok = _close(lg, r.logits[:, -1], 2e-2)
        assert ok, err
        dec.resize(200)  # grow capacity mid-conversation: K/V survive, graphs are re-captured
        pk, t = r.past_key_values, r.logits[:, -1].argmax(-1)
        for _ in range(3):
            rr = ref(input_ids=t[:, None], past_key_values=pk, use_cache=True)
            pk = rr.past_key_values
            err, ok = _close(dec.next(t.cuda()), rr.logits[:, -1], 2e-2)
            assert ok, err
            t = rr.logits[:, -1].argmax(-1)
    rt.cache.free()


def test_paged_block_fused_paths_agree():
    """PagedMoEBlock for one token: the two-kernel path (fused=2), the per-expert path
    (fused=1) and the dequant + GEMM path (fused=0) give the same layer output."""
    cfg, ref, gpu, rt = _models(seed=7, nslots=24)
    blk = gpu.model.layers[1].mlp
    x = torch.randn(1, 1, H, device="cuda").to(torch.bfloat16)
    outs = {}
    with torch.no_grad():
        for f in (2, 1, 0):
            rt.fused = f
            y = blk(x)
            outs[f] = (y[0] if isinstance(y, tuple) else y).float()
    for f in (1, 0):
        err = ((outs[f] - outs[2]).norm() / outs[2].norm()).item()
        assert err <= 1e-2, (f, err)
    rt.cache.free()
