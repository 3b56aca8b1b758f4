"""GPU parity: attention block (qkv 2-bit projection, qk-norm + RoPE, KV append, windowed
chain/tree SDPA, o-projection with residual) vs the oracle's attention block."""
import numpy as np
import pytest

from momij_amd import synth
from tests.gpu_util import assert_close, dev, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from momij_amd.ops import Context

    c = Context(0)
    yield c
    c.close()


TREE16 = [-1, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 10, 11, 12, 13, 14]  # 16 nodes, depth 6


@pytest.mark.parametrize("case", ["cfg2_chain", "ring_wrap", "tree16", "rope128", "full_attn",
                                  "early_window", "ring_shared_chunk", "ring_tree16"])
def test_attn_block(ctx, orc, case):
    import torch

    print(f"case: attn {case}", flush=True)
    rng = np.random.default_rng(abs(hash(case)) % 10000)
    H, nQ, nKV, D, gs = 2048, 16, 4, 128, 64
    cfg = dict(H=H, nQ=nQ, nKV=nKV, D=D, rope_dim=64, rope_base=1e6, eps=1e-6, window=1024,
               C=4096 + 64, gs=gs)
    L, parents = 4096, list(range(-1, 8))  # K=8 chain -> 9 rows ([y] + 8 drafts)
    if case == "ring_wrap":
        cfg["C"], L = 1024 + 64, 5000
    elif case == "ring_shared_chunk":
        # the window's first keys and the pass's last rows sit in one 64-slot chunk of the ring
        # (the 56 unused slots between them: (L + 8) % C = 194 = 3 * 64 + 2)
        cfg["C"], L = 1024 + 64, 4538
    elif case == "ring_tree16":
        cfg["C"], L, parents = 1024 + 64, 4538, TREE16
    elif case == "tree16":
        parents = TREE16
    elif case == "rope128":
        cfg["rope_dim"] = 128
    elif case == "full_attn":
        cfg["window"], L, cfg["C"] = 0, 700, 1024
    elif case == "early_window":
        L = 300  # fewer committed tokens than the window
    M = len(parents)
    aw = synth.attn_weights(rng, H, nQ, nKV, D, gs)
    h = synth.normal_f16(rng, (M, H))
    kc = synth.normal_f16(rng, (nKV, cfg["C"], D))
    vc = synth.normal_f16(rng, (nKV, cfg["C"], D))
    ref_h, ref_k, ref_v = orc.attn_block(cfg, aw, h, kc, vc, L, np.array(parents, np.int32))
    daw = {k: dev(v) for k, v in aw.items()}
    dh, dk, dv = dev(h), dev(kc), dev(vc)
    torch.cuda.synchronize()
    ctx.attn_block(cfg, daw, dh, dk, dv, L, parents, M)
    ctx.sync()
    rel, _ = assert_close(host(dh), ref_h, what=f"{case} h")
    assert rel < 5e-3
    slots = [(L + r) % cfg["C"] for r in range(M)]
    assert_close(host(dk)[:, slots], ref_k[:, slots], what=f"{case} new K")
    assert_close(host(dv)[:, slots], ref_v[:, slots], what=f"{case} new V")
    # untouched slots stay untouched
    other = [s for s in range(0, cfg["C"], 97) if s not in slots]
    assert (host(dk)[:, other].view(np.uint16) == kc[:, other].view(np.uint16)).all()


def test_tree_chain_equals_chain(ctx):
    """A tree whose nodes form one chain reproduces the chain pass bit for bit."""
    import torch

    rng = np.random.default_rng(42)
    H, nQ, nKV, D, gs = 2048, 16, 4, 128, 64
    cfg = dict(H=H, nQ=nQ, nKV=nKV, D=D, rope_dim=64, rope_base=1e6, eps=1e-6, window=256,
               C=256 + 64, gs=gs)
    M, L = 7, 1000
    aw = {k: dev(v) for k, v in synth.attn_weights(rng, H, nQ, nKV, D, gs).items()}
    h = synth.normal_f16(rng, (M, H))
    kc = synth.normal_f16(rng, (nKV, cfg["C"], D))
    vc = synth.normal_f16(rng, (nKV, cfg["C"], D))
    outs = []
    for parents in (None, list(range(-1, M - 1))):
        dh, dk, dv = dev(h), dev(kc), dev(vc)
        torch.cuda.synchronize()
        ctx.attn_block(cfg, aw, dh, dk, dv, L, parents, M)
        ctx.sync()
        outs.append(host(dh).view(np.uint16))
    assert (outs[0] == outs[1]).all()
