"""The benchmark configurations at their own shapes, checked against the oracle.

C3 -- all 128 experts of the layer at 3 and 2 bits: quantizer bytes and dequantized bf16
bit-exact with the oracle.

C5 -- grouped prefill, H=2048, I=768, 128 experts, top-8, T = 64 / 256 / 512 tokens routed
by Zipf(1.1) as the benchmark draws them, against the binary64 restatement of the
reference's per-expert dequant + F.linear path (moe.py:131-151, oracle.moe_prefill_f64).

C4 -- the full 48-layer Qwen3-30B-A3B-shaped decode step (Hq 32, Hk 4, head_dim 128,
H 2048, 128 experts of I 768, top-8, KV length 4096) with a random-init skeleton, 4-bit
experts in a pinned host store, a 512-slot LRU cache and Zipf(1.1) expert draws, over 5
decode tokens (the pattern of the reference's tests/test_graphdec.py:49-83):
  * graph replay and eager execution give bit-identical logits every token;
  * the cache's bookkeeping equals the reference LRU (oracle/cache_core_ref.py) on the same
    key stream, and every resident slot holds exactly its store row;
  * the MoE output of sampled layers equals the binary64 oracle of the fused layer on the
    slot contents the kernels read, within the 1e-3 bar.
To keep the store's build short, layer l's experts hold the same bytes as layer 0's (the
store still has all 48 x 128 rows, 15.4 GB pinned, and the cache pages each row by its
own key).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle.cache_core_ref import RefCore
from wisp import kernels

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, I, E, K, G = 2048, 768, 128, 8, 128


def _zipf_experts(rng, k, s, perm):
    """k distinct experts: Zipf(s) over ranks 1..E by Gumbel-top-k, mapped through perm."""
    g = rng.gumbel(size=E) - s * np.log(np.arange(1, E + 1))
    return perm[np.argsort(-g)[:k]]


def _gpu_pool(E_, bits, seed):
    """E_ experts quantized on the GPU (the bit-exact quantizer) -> (device pool, host copy)."""
    from wisp.quant import expert_nbytes, quantize

    gen = torch.Generator(device=DEV).manual_seed(seed)
    pool = torch.empty((E_, expert_nbytes(H * I, bits, G)), dtype=torch.uint8, device=DEV)
    for e in range(E_):
        quantize(torch.randn((3, H * I), generator=gen, device=DEV) * 0.02, bits, G, out=pool[e])
    return pool, pool.cpu().numpy()


# ---------------------------------------------------------------- C3
@pytest.mark.parametrize("bits", [3, 2])
def test_c3_quantize_and_dequant_bit_exact_for_all_128_experts(bits):
    """C3's check: 128 experts of the Qwen3 shape quantized on the GPU, every byte equal to
    the oracle quantizer's (quant.py:60-73), and dequantized on the GPU, every bf16 equal to
    the oracle's unpack and dequant (quant.py:76-87). Weights drawn on the GPU in blocks of
    16 experts and copied to the host for the oracle."""
    from wisp import quant

    n = H * I
    gen = torch.Generator(device=DEV).manual_seed(300 + bits)
    nb = quant.expert_nbytes(n, bits, G)
    for e0 in range(0, E, 16):
        w = torch.randn((16, 3, n), generator=gen, device=DEV) * 0.02
        rows = torch.empty((16, nb), dtype=torch.uint8, device=DEV)
        for j in range(16):
            quant.quantize(w[j], bits, G, out=rows[j])
        got_rows = rows.cpu().numpy()
        w_host = w.cpu().numpy()
        for j in range(16):
            assert np.array_equal(got_rows[j], O.quantize(w_host[j], bits, G)), (bits, e0 + j)
        deq = quant.dequant(rows, n, bits, G)
        torch.cuda.synchronize()
        assert np.array_equal(deq.view(torch.int16).cpu().numpy().view(np.uint16), O.dequant(got_rows, n, bits, G)), \
            (bits, e0)
        del w, rows, deq


# ---------------------------------------------------------------- C5
@pytest.fixture(scope="module")
def c5_pool():
    return _gpu_pool(E, 4, seed=55)


@pytest.mark.parametrize("T", [64, 256, 512])
def test_c5_prefill_full_shape_zipf(c5_pool, T):
    pool, pool_np = c5_pool
    rng = np.random.default_rng(T)
    perm = rng.permutation(E)
    sel = np.stack([_zipf_experts(rng, K, 1.1, perm) for _ in range(T)]).astype(np.int64)
    rw = O.bf16_bits_to_f32(O.f32_to_bf16_bits(rng.random((T, K)).astype(np.float32))).reshape(T, K)
    x = O.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32)).reshape(T, H)
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV)
    out = kernels.moe_prefill(pool, {e: e for e in range(E)}, xt, torch.from_numpy(sel),
                              torch.from_numpy(rw).to(DEV), H * I, H, I, 4)
    torch.cuda.synchronize()
    ref = O.moe_prefill_f64(pool_np, {e: e for e in range(E)}, x, sel, rw, H, I, 4)
    r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32))).reshape(ref.shape)
    got = out.float().cpu().numpy()
    err = np.linalg.norm(got - r) / np.linalg.norm(r)
    print(f"C5 T={T}: {len(np.unique(sel))} experts, rel-L2 {err:.3e}")
    assert err <= 1e-3, err


def test_c5_prefill_3bit_t256():
    pool, pool_np = _gpu_pool(E, 3, seed=56)
    rng = np.random.default_rng(9)
    T = 256
    sel, rw = O.route(rng.standard_normal((T, E)).astype(np.float32), K)
    x = O.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32)).reshape(T, H)
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV)
    out = kernels.moe_prefill(pool, {e: e for e in range(E)}, xt, torch.from_numpy(sel),
                              torch.from_numpy(rw).to(DEV), H * I, H, I, 3)
    ref = O.moe_prefill_f64(pool_np, {e: e for e in range(E)}, x, sel, rw, H, I, 3)
    r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32))).reshape(ref.shape)
    err = np.linalg.norm(out.float().cpu().numpy() - r) / np.linalg.norm(r)
    print(f"C5 3-bit T=256: rel-L2 {err:.3e}")
    assert err <= 1e-3, err


# ---------------------------------------------------------------- C4
C4_LAYERS, C4_SLOTS, C4_TMAX, C4_TOKENS, C4_POS0 = 48, 512, 4096, 5, 4000
SAMPLED = (0, 17, 47)


def _c4_config():
    from transformers import Qwen3MoeConfig

    return Qwen3MoeConfig(vocab_size=151936, hidden_size=H, intermediate_size=6144, moe_intermediate_size=I,
                          num_hidden_layers=C4_LAYERS, num_attention_heads=32, num_key_value_heads=4, head_dim=128,
                          num_experts=E, num_experts_per_tok=K, norm_topk_prob=True, rms_norm_eps=1e-6,
                          rope_theta=1e6, max_position_embeddings=40960, decoder_sparse_step=1, mlp_only_layers=[])


@pytest.fixture(scope="module")
def c4_setup():
    pytest.importorskip("transformers")
    from wisp.model import random_skeleton
    from wisp.moe import Runtime
    from wisp.store import ExpertStore

    store = ExpertStore(C4_LAYERS, E, H * I, 4, G)
    base, _ = _gpu_pool(E, 4, seed=44)
    host0 = base.cpu()
    for l in range(C4_LAYERS):  # layer l's rows hold layer 0's bytes (see the module docstring)
        store.host[l * E:(l + 1) * E].copy_(host0)
    del base
    rt = Runtime(store, fused=2)
    model = random_skeleton(_c4_config(), rt, device=DEV)
    rng = np.random.default_rng(4)
    perms = [rng.permutation(E) for _ in range(C4_LAYERS)]
    draws = [[_zipf_experts(rng, K, 1.1, perms[i]).astype(np.int64) for i in range(C4_LAYERS)]
             for _ in range(C4_TOKENS)]
    g = torch.Generator(device=DEV).manual_seed(12)
    kv0 = torch.randn((C4_LAYERS, 2, 4, C4_POS0, 128), generator=g, device=DEV).to(torch.bfloat16)
    return store, rt, model, draws, kv0


def _decode(c4_setup, use_graph, device_paging=False):
    """C4_TOKENS greedy decode tokens after a random context of C4_POS0 positions; returns the
    logits of each token, the decoder, and the sampled layers' (x, meta, slot rows, output)."""
    from wisp.cache import ExpertCache
    from wisp.graphdec import GraphDecoder

    store, rt, model, draws, kv0 = c4_setup
    if rt.cache is not None:
        rt.cache.free()
    rt.cache = ExpertCache(store, C4_SLOTS)
    rt.reset_stats()
    samples = []

    class ZipfDecoder(GraphDecoder):
        def _expert_ids(self, i):
            return draws[self.pos - C4_POS0][i]

        def _moe(self, i):
            y = super()._moe(i)
            if not use_graph and i in SAMPLED:  # eager: record what the kernels read and wrote
                slots = self.meta_dev[:K].to(torch.int64)
                samples.append((self.pos, i, self.xn.view(-1).clone(), self.meta_dev.clone(),
                                self.rt.cache.gpu.index_select(0, slots).clone(), y.clone()))
            return y

    dec = ZipfDecoder(model, rt, tmax=C4_TMAX, use_graph=use_graph, device_paging=device_paging)
    with torch.no_grad():
        dec.kv[:, :, :, :C4_POS0].copy_(kv0)
        dec.pos = C4_POS0
        tok = torch.zeros(1, dtype=torch.long, device=DEV)
        logits = []
        for _ in range(C4_TOKENS):
            lg = dec.next(tok).clone()
            logits.append(lg)
            tok = lg.argmax(-1)
    torch.cuda.synchronize()
    return torch.stack(logits), dec, samples


def test_c4_full_shape_graph_equals_eager_and_cache_matches_reference(c4_setup):
    store, rt, model, draws, kv0 = c4_setup
    eager, _, samples = _decode(c4_setup, use_graph=False)
    core_eager = rt.cache.core
    where_eager = dict(core_eager.key2slot)
    graph, dec, _ = _decode(c4_setup, use_graph=True)
    assert dec.graphs is not None and len(dec.graphs) == C4_LAYERS + 1
    assert torch.isfinite(graph.float()).all()
    assert torch.equal(graph.view(torch.int16), eager.view(torch.int16)), "graph replay differs from eager"

    # the cache's bookkeeping vs the reference LRU on the same key stream (both runs)
    ref = RefCore(C4_SLOTS, "lru")
    for t in range(C4_TOKENS):
        for i in range(C4_LAYERS):
            ref.ensure([i * E + int(e) for e in draws[t][i]])
    core = rt.cache.core
    assert core.key2slot == ref.where and where_eager == ref.where
    st = core.stats
    assert {n: st[n] for n in ("hits", "misses", "evictions")} == {n: ref.counts[n] for n in ("hits", "misses",
                                                                                              "evictions")}
    assert st["hits"] + st["misses"] == C4_TOKENS * C4_LAYERS * K and st["misses"] > 0
    print(f"C4: {st['hits']} hits, {st['misses']} misses, {st['evictions']} evictions")

    # every resident slot holds exactly its store row
    items = sorted(core.key2slot.items())
    for c0 in range(0, len(items), 64):
        keys = [kk for kk, _ in items[c0:c0 + 64]]
        slots = torch.tensor([ss for _, ss in items[c0:c0 + 64]], device=DEV)
        got = rt.cache.gpu.index_select(0, slots).cpu()
        assert torch.equal(got, store.host[keys]), keys[:4]

    # the sampled layers' MoE output against the binary64 oracle on the slot contents
    assert len(samples) == C4_TOKENS * len(SAMPLED)
    for pos, i, x, meta, rows, y in samples:
        rows_np = rows.cpu().numpy()
        w = meta[K:].cpu().numpy()
        xb = x.view(torch.int16).cpu().numpy().view(np.uint16)
        _, _, r64 = O.moe_layer_f64(rows_np, np.arange(K), w, xb, H, I, 4, G)
        r = O.bf16_bits_to_f32(O.f32_to_bf16_bits(r64.astype(np.float32))).astype(np.float64)
        got = y.float().cpu().numpy().astype(np.float64)
        err = float(np.linalg.norm(got - r) / np.linalg.norm(r))
        print(f"C4 pos {pos} layer {i}: MoE rel-L2 {err:.3e}")
        assert err <= 1e-3, (pos, i, err)

    # the same decode with the paging points on the GPU: one graph per token, the same
    # logits bit for bit and the same LRU bookkeeping
    dgraph, ddec, _ = _decode(c4_setup, use_graph=True, device_paging=True)
    assert ddec._dev and len(ddec.graphs) == 1
    assert torch.equal(dgraph.view(torch.int16), eager.view(torch.int16)), "device paging differs from eager"
    core = rt.cache.core
    assert core.key2slot == ref.where
    assert {n: core.stats[n] for n in ("hits", "misses", "evictions", "calls")} == {
        n: ref.counts[n] for n in ("hits", "misses", "evictions", "calls")}
    items = sorted(core.key2slot.items())
    for c0 in range(0, len(items), 64):
        keys = [kk for kk, _ in items[c0:c0 + 64]]
        slots = torch.tensor([ss for _, ss in items[c0:c0 + 64]], device=DEV)
        assert torch.equal(rt.cache.gpu.index_select(0, slots).cpu(), store.host[keys]), keys[:4]
    rt.cache.free()
    rt.cache = None
