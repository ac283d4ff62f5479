"""gpt-oss experts on the GPU (wisp/gptoss.py): the MXFP4 decoder and the fused decode
kernels against the CPU oracle, and the paged block against transformers' GptOssMLP.

Bars: MXFP4 -> bf16 bit-exact; the fused decode layer within 1e-3 relative L2 of the
oracle (oracle.gptoss_block_ref: bit-exact bf16 weights, binary64 GEMVs, the
reference's bf16 rounding of each intermediate tensor); the paged block within the
reference's own criteria against transformers (tests/test_gptoss.py:69-78: 5 % of the
max output with 16-bit experts, 35 % with 4-bit).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from wisp import kernels

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bits16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


# ---------------------------------------------------------------- MXFP4
def test_mxfp4_every_byte_and_scale():
    # all 256 block bytes under all 256 scale bytes (incl. the subnormal 2^-127 and inf)
    blocks = np.tile(np.arange(256, dtype=np.uint8).reshape(16, 16), (256, 1, 1))  # [256 scales, 16, 16]
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 16, 1)              # [256, 16]
    got = kernels.mxfp4_to_bf16(torch.from_numpy(blocks).to(DEV), torch.from_numpy(scales).to(DEV))
    torch.cuda.synchronize()
    assert got.shape == (256, 512)
    assert np.array_equal(_bits16(got), O.mxfp4_to_bf16_bits(blocks, scales))


def test_mxfp4_random_large():
    rng = np.random.default_rng(3)
    blocks = rng.integers(0, 256, (4, 96, 90, 16), dtype=np.uint8)
    scales = rng.integers(110, 135, (4, 96, 90), dtype=np.uint8)
    got = kernels.mxfp4_to_bf16(torch.from_numpy(blocks).to(DEV), torch.from_numpy(scales).to(DEV))
    assert np.array_equal(_bits16(got), O.mxfp4_to_bf16_bits(blocks, scales))


# ---------------------------------------------------------------- fused decode
def _gptoss_case(E, H, I, k, bits, group, seed, wscale=0.05):
    rng = np.random.default_rng(seed)
    n = H * I
    pool = np.stack([O.quantize((rng.standard_normal(3 * n) * wscale).astype(np.float32), bits, group)
                     for _ in range(E)])
    gub = O.f32_to_bf16_bits((rng.standard_normal((E, 2 * I)) * 0.5).astype(np.float32)).reshape(E, 2 * I)
    db = O.f32_to_bf16_bits((rng.standard_normal((E, H)) * 0.5).astype(np.float32)).reshape(E, H)
    x = O.f32_to_bf16_bits((rng.standard_normal(H) * 2.0).astype(np.float32)).reshape(1, H)
    ex = rng.permutation(E)[:k]
    logits = torch.from_numpy(rng.standard_normal((1, k)).astype(np.float32)).to(torch.bfloat16)
    sc = torch.softmax(logits, dim=1, dtype=torch.bfloat16).float().numpy()
    slots = rng.permutation(E)  # expert e lives in slot slots[e]
    pool_by_slot = np.empty_like(pool)
    pool_by_slot[slots] = pool
    return pool_by_slot, slots, gub, db, x, ex.reshape(1, k), sc


def _run_decode(pool, slots, gub, db, x, ex, sc, H, I, bits, group, meta_override=None):
    k = ex.shape[1]
    meta = np.concatenate([slots[ex[0]].astype(np.float32), sc[0], ex[0].astype(np.float32)])
    if meta_override is not None:
        meta = meta_override(meta)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    out = kernels.gptoss_decode(t(pool), t(meta), t(x.view(np.int16)).view(torch.bfloat16).reshape(-1),
                                t(gub.view(np.int16)).view(torch.bfloat16), t(db.view(np.int16)).view(torch.bfloat16),
                                k, H * I, H, I, bits, group)
    torch.cuda.synchronize()
    return O.bf16_bits_to_f32(_bits16(out))


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("E,H,I,k,group", [(8, 64, 64, 2, 64),      # the reference's test shape
                                           (6, 256, 256, 4, 128),
                                           (5, 2880, 2880, 4, 128),  # gpt-oss-20b: down rows straddle groups
                                           (4, 320, 160, 3, 32),     # H != I (kernel-level), partial blocks
                                           (20, 96, 48, 12, 32),     # H % 64 == 32: a partial gate_up row block;
                                                                     # k > 8: several batches of 8 experts
                                           (18, 256, 256, 9, 128),
                                           (18, 256, 256, 16, 128)])
def test_gptoss_decode_matches_oracle(bits, E, H, I, k, group):
    pool, slots, gub, db, x, ex, sc = _gptoss_case(E, H, I, k, bits, group, seed=H + bits)
    got = _run_decode(pool, slots, gub, db, x, ex, sc, H, I, bits, group)
    ref = O.bf16_bits_to_f32(O.gptoss_block_ref(pool, {int(e): int(slots[e]) for e in range(E)}, x, ex, sc,
                                                 gub, db, H, I, bits, group))[0]
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    print(f"gptoss decode bits={bits} H={H} I={I} k={k}: rel-L2 {err:.3e}")
    assert np.isfinite(got).all()
    assert err <= 1e-3, err


def test_gptoss_decode_invalid_ids_poison_the_output():
    E, H, I, k, bits, group = 6, 256, 256, 3, 4, 128
    pool, slots, gub, db, x, ex, sc = _gptoss_case(E, H, I, k, bits, group, seed=9)

    def bad_slot(m):
        m = m.copy()
        m[1] = 99.0
        return m

    def bad_expert(m):
        m = m.copy()
        m[2 * k] = 1.5
        return m

    for f in (bad_slot, bad_expert):
        got = _run_decode(pool, slots, gub, db, x, ex, sc, H, I, bits, group, meta_override=f)
        assert np.isnan(got).all()
    ok = _run_decode(pool, slots, gub, db, x, ex, sc, H, I, bits, group)
    assert np.isfinite(ok).all()


def test_gptoss_decode_graph_follows_meta():
    # the kernels read slot ids, weights and expert ids from device memory at run time
    E, H, I, k, bits, group = 6, 256, 256, 2, 4, 128
    pool, slots, gub, db, x, ex, sc = _gptoss_case(E, H, I, k, bits, group, seed=21)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    pool_d, gub_d, db_d = t(pool), t(gub.view(np.int16)).view(torch.bfloat16), t(db.view(np.int16)).view(torch.bfloat16)
    x_d = t(x.view(np.int16)).view(torch.bfloat16).reshape(-1)
    meta_d = torch.zeros(3 * k, dtype=torch.float32, device=DEV)
    routes = [(np.array([[0, 3]]), np.array([[0.75, 0.25]], np.float32)),
              (np.array([[5, 1]]), np.array([[0.5, 0.5]], np.float32))]
    for e_, s_ in routes:  # warm-up outside the capture
        meta_d.copy_(t(np.concatenate([slots[e_[0]].astype(np.float32), s_[0], e_[0].astype(np.float32)])))
        kernels.gptoss_decode(pool_d, meta_d, x_d, gub_d, db_d, k, H * I, H, I, bits, group)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = kernels.gptoss_decode(pool_d, meta_d, x_d, gub_d, db_d, k, H * I, H, I, bits, group)
    for _ in range(2):
        for e_, s_ in routes:
            meta_d.copy_(t(np.concatenate([slots[e_[0]].astype(np.float32), s_[0], e_[0].astype(np.float32)])))
            g.replay()
            torch.cuda.synchronize()
            ref = O.bf16_bits_to_f32(O.gptoss_block_ref(pool, {int(e): int(slots[e]) for e in range(E)}, x, e_, s_,
                                                         gub, db, H, I, bits, group))[0]
            got = O.bf16_bits_to_f32(_bits16(out))
            assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-3


# ---------------------------------------------------------------- paged block vs transformers
def _hf_block(N, seed=1):
    from transformers import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssMLP

    torch.manual_seed(seed)
    cfg = GptOssConfig(hidden_size=64, intermediate_size=64, num_hidden_layers=1, num_local_experts=8,
                       num_experts_per_tok=2, num_attention_heads=2, num_key_value_heads=1, head_dim=32, vocab_size=50)
    ref = GptOssMLP(cfg).to(torch.bfloat16)  # stays on the CPU: the reference runs its test there
    with torch.no_grad():
        for p in ref.parameters():
            p.normal_(0, 0.3)
    x = torch.randn(1, N, 64).to(torch.bfloat16)
    return cfg, ref, x


def _paged_block(cfg, ref, bits, group=64):
    from wisp.cache import ExpertCache
    from wisp.gptoss import PagedGptOssBlock, expert_w3
    from wisp.moe import Runtime
    from wisp.store import ExpertStore

    E, H, I = 8, 64, 64
    st = ExpertStore(1, E, H * I, bits, group, pin=True)
    for e in range(E):
        st.put(0, e, expert_w3(ref.experts.gate_up_proj[e].data, ref.experts.down_proj[e].data), DEV)
    rt = Runtime(st, ExpertCache(st, nslots=E, device=DEV))
    router = torch.nn.Linear(H, E, bias=True, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        router.weight.copy_(ref.router.weight.data)
        router.bias.copy_(ref.router.bias.data)
    blk = PagedGptOssBlock(router, 0, rt, cfg, device=DEV)
    blk.gub.copy_(ref.experts.gate_up_proj_bias.data)
    blk.db.copy_(ref.experts.down_proj_bias.data)
    return blk, rt


@pytest.mark.parametrize("bits,frac", [(16, 0.05), (4, 0.35)])
@pytest.mark.parametrize("N", [1, 5])
def test_paged_block_close_to_transformers(bits, frac, N):
    cfg, ref, x = _hf_block(N)
    blk, rt = _paged_block(cfg, ref, bits)
    with torch.no_grad():
        want, _ = ref(x)
        got, sc = blk(x.to(DEV))
    got = got.cpu()
    d, m = (got.float() - want.float()).abs().max().item(), want.float().abs().max().item()
    print(f"paged gpt-oss block bits={bits} N={N}: max|d| {d:.3e} of max {m:.3e}")
    assert got.shape == want.shape and sc.shape == (N, 2)
    assert d < frac * m, (d, m)
    assert rt.stats["gpu_experts"] >= 2


def test_paged_block_fused_decode_matches_dequant_path():
    # one token, 4-bit: the fused kernels and the reference's dequantize + bmm path are two
    # implementations of the same bf16 semantics
    cfg, ref, x = _hf_block(1, seed=4)
    blk, rt = _paged_block(cfg, ref, 4)
    with torch.no_grad():
        fused, _ = blk(x.to(DEV))
        blk._fused_ok = lambda cache: False  # this block instance takes the dequantize + bmm path
        slow, _ = blk(x.to(DEV))
    err = ((fused.float() - slow.float()).norm() / slow.float().norm()).item()
    print(f"gpt-oss fused vs dequant path: rel-L2 {err:.3e}")
    assert err <= 1e-2
