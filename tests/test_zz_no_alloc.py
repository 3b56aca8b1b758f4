"""GPU check of mj_moe_block_noalloc (the MoE block over the library's static per-GPU scratch)
against mj_moe_block on the same inputs: two calls in a row, the second with fewer rows, both
bit for bit equal (the same kernels); a shape whose scratch exceeds MJ_MOE_NOALLOC_BYTES is
refused with MJ_CAPACITY before any work is queued."""
import numpy as np
import pytest

from momij_amd import synth
from tests.gpu_util import dev, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from momij_amd.ops import Context

    c = Context(0)
    yield c
    c.close()


def _moe_dev(rng, E, H, I, gs, k):
    mw = synth.moe_weights(rng, E, H, I, gs, top_k=k)
    return {kk: (dev(v) if isinstance(v, np.ndarray) else v) for kk, v in mw.items()}


@pytest.mark.parametrize("E,gs", [(64, 64), (256, 128)])
def test_noalloc_equals_moe_block(ctx, E, gs):
    import torch

    rng = np.random.default_rng(E + gs)
    H, I, k = 2048, 1024, 8
    dmw = _moe_dev(rng, E, H, I, gs, k)
    for M in (17, 3):  # the second call has fewer rows than the first
        print(f"case: moe_block_noalloc E={E} gs={gs} M={M}", flush=True)
        x = dev(synth.normal_f16(rng, (M, H)))
        outs = []
        for fn in (ctx.moe_block, ctx.moe_block_noalloc):
            y = torch.empty_like(x)
            inds = torch.full((M, k), -1, dtype=torch.int32, device="cuda")
            scores = torch.zeros((M, k), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            fn(dmw, x, y, M, 3, inds, scores)
            ctx.sync()
            outs.append((host(y), host(inds), host(scores)))
        (y0, i0, s0), (y1, i1, s1) = outs
        assert (i0 == i1).all() and (s0.view(np.uint32) == s1.view(np.uint32)).all()
        assert (y0.view(np.uint16) == y1.view(np.uint16)).all()


def test_noalloc_refuses_oversized_scratch(ctx):
    import torch

    from momij_amd._lib import MomijError

    # H = I = 4096 at 64 rows needs about 9.5 MB of scratch: refused before any launch
    print("case: moe_block_noalloc refusal H=4096 I=4096 M=64", flush=True)
    rng = np.random.default_rng(3)
    E, H, I, gs, k, M = 8, 4096, 4096, 64, 8, 64
    dmw = _moe_dev(rng, E, H, I, gs, k)
    x = dev(synth.normal_f16(rng, (M, H)))
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    with pytest.raises(MomijError) as ei:
        ctx.moe_block_noalloc(dmw, x, y, M, 3)
    assert ei.value.status == 7 and "MJ_MOE_NOALLOC_BYTES" in str(ei.value)
    ctx.sync()
