"""esc_moe_expert_path_static (the expert path with its scratch in the
library's device array, no allocation in the call) against esc_moe_expert_path
(caller workspace), through the C-ABI.

Both run the same kernels on the same inputs, so their outputs must be
bit-identical.  The static array keeps the previous call's contents: the calls
run in a row with shapes that shrink (and a shape of the other kernel path in
between), so a counter left where another shape keeps data would show.  The
order-exact chain and the oracle pin the regular entry point elsewhere; here
the expert path's output is also held to the oracle at one shape.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_np as R

from .conftest import has_gpu

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not has_gpu(), reason="needs a ROCm GPU")]

DEV = "cuda"


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[gpu case] {request.node.nodeid}", flush=True)
    yield
    torch.cuda.synchronize()


def _case(E, H, I, T, k, seed):
    rng = np.random.default_rng(seed)
    u32 = lambda *s: rng.integers(0, 2**32, size=s, dtype=np.uint64).astype(np.uint32)
    c = dict(gu_code=u32(E, H // 16, 2 * I // 16, 16), dn_code=u32(E, I // 16, H // 16, 16),
             gu_rin=rng.choice([-1.0, 1.0], (E, H)).astype(np.float32),
             dn_rin=rng.choice([-1.0, 1.0], (E, I)).astype(np.float32),
             gu_rout=(rng.choice([-1.0, 1.0], (E, 2 * I)) * rng.uniform(0.5, 1.5, (E, 2 * I))
                      * 4e-2).astype(np.float32),
             dn_rout=(rng.choice([-1.0, 1.0], (E, H)) * rng.uniform(0.5, 1.5, (E, H))
                      * 4e-2).astype(np.float32),
             x=rng.standard_normal((T, H)).astype(np.float16),
             logits=rng.standard_normal((T, E)).astype(np.float32))
    return c


def _device(c, k):
    from escha_mlx_amd import ops
    d = {n: torch.from_numpy(np.ascontiguousarray(v)).to(DEV) for n, v in c.items()}
    d["gu_code"] = d["gu_code"].view(torch.int32)
    d["dn_code"] = d["dn_code"].view(torch.int32)
    d["ids"], d["scores"] = ops.route_topk(d["logits"], k)
    return d


def _both(d, K=2, lut=None):
    """(static entry point's output, regular entry point's output)."""
    from escha_mlx_amd import ops
    args = (d["x"], d["ids"], d["scores"], d["gu_code"], d["gu_rin"], d["gu_rout"], K,
            d["dn_code"], d["dn_rin"], d["dn_rout"], K)
    y_s = torch.full(tuple(d["x"].shape), float("nan"), dtype=torch.float16, device=DEV)
    ops.moe_expert_path_static(*args, out=y_s, lut=lut)
    y_r = ops.moe_expert_path(*args, lut=lut)
    return y_s, y_r


def test_static_expert_path_equals_workspace_path_in_a_row():
    """Two calls in a row at config 3's expert shape (E=256, H=2048, I=512,
    top-8, K=2), the second with fewer tokens, then a shape of the one
    persistent launch, then the first shape again: each bit-identical to the
    workspace entry point."""
    from escha_mlx_amd import ops
    k = 8
    big = _device(_case(256, 2048, 512, 4, k, 901), k)
    small = _device(_case(256, 2048, 512, 1, k, 902), k)
    other = _device(_case(64, 512, 256, 2, k, 903), k)
    for name, d in (("T=4", big), ("T=1", small), ("persistent T=2", other), ("T=4 again", big),
                    ("T=1 again", small)):
        y_s, y_r = _both(d)
        torch.cuda.synchronize()
        assert not torch.isnan(y_s.float()).any(), name
        assert torch.equal(y_s.view(torch.int16), y_r.view(torch.int16)), name


def test_static_expert_path_vs_oracle():
    """The static call's output at T=1 against the oracle's routed block."""
    E, H, I, k = 256, 2048, 512, 8
    c = _case(E, H, I, 1, k, 904)
    d = _device(c, k)
    y_s, _ = _both(d)
    ids, sc = d["ids"].cpu().numpy(), d["scores"].cpu().numpy()
    w_gu = np.zeros((E, H, 2 * I), np.float16)
    w_dn = np.zeros((E, I, H), np.float16)
    for e in np.unique(ids):
        w_gu[e] = R.reconstruct(c["gu_code"][e], H, 2 * I, 2)
        w_dn[e] = R.reconstruct(c["dn_code"][e], I, H, 2)
    want = R.moe_routed(c["x"], ids, sc, {"w": w_gu, "rin": c["gu_rin"], "rout": c["gu_rout"]},
                        {"w": w_dn, "rin": c["dn_rin"], "rout": c["dn_rout"]}, 2, 2,
                        ordered=True).astype(np.float32)
    got = y_s.cpu().numpy().astype(np.float32)
    assert np.abs(got - want).max() / np.abs(want).max() < 5e-3


def test_static_expert_path_rejects_oversize():
    """A shape whose plan needs more than the array holds is refused with a
    clear error and leaves the array usable."""
    from escha_mlx_amd import ops
    k = 8
    huge = _device(_case(256, 2048, 512, 48, k, 905), k)
    y = torch.empty((48, 2048), dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError, match="workspace|counter region"):
        ops.moe_expert_path_static(huge["x"], huge["ids"], huge["scores"], huge["gu_code"],
                                   huge["gu_rin"], huge["gu_rout"], 2, huge["dn_code"],
                                   huge["dn_rin"], huge["dn_rout"], 2, out=y)
    small = _device(_case(256, 2048, 512, 1, k, 906), k)
    y_s, y_r = _both(small)
    assert torch.equal(y_s.view(torch.int16), y_r.view(torch.int16))
    assert ops.moe_expert_path_static_max() == 4 << 20


def _args(d, K=2):
    return (d["x"], d["ids"], d["scores"], d["gu_code"], d["gu_rin"], d["gu_rout"], K,
            d["dn_code"], d["dn_rin"], d["dn_rout"], K)


def test_static_grouped_shape_between_fused_shapes():
    """More than 64 routed rows at small H and I (E=8, H=512, I=256, 16
    tokens, top-8: the grouped split-K chain, whose data starts after the
    counter region) between two calls of the two-launch path and one of the
    persistent launch, each bit-identical to the workspace entry point."""
    k = 8
    fused = _device(_case(256, 2048, 512, 1, k, 910), k)
    grouped = _device(_case(8, 512, 256, 16, k, 911), k)
    pers = _device(_case(64, 512, 256, 2, k, 912), k)
    for name, d in (("two-launch T=1", fused), ("grouped T=16", grouped), ("persistent T=2", pers),
                    ("grouped again", grouped), ("two-launch again", fused)):
        y_s, y_r = _both(d)
        torch.cuda.synchronize()
        assert not torch.isnan(y_s.float()).any(), name
        assert torch.equal(y_s.view(torch.int16), y_r.view(torch.int16)), name


def test_static_grouped_table_shape_equals_workspace_path():
    """The grouped chain with the table asked for (the persistent
    k_gemv_rows_table, whose item count it reads from the scratch) through
    the static array, bit-identical to the workspace entry point, between two
    calls of the grouped chain by hash."""
    from escha_mlx_amd import ops
    ops.init()
    k = 8
    grouped = _device(_case(8, 512, 256, 16, k, 913), k)
    other = _device(_case(16, 512, 256, 16, k, 914), k)  # within the 4 MiB scratch
    for name, d, lut in (("hash E=8", grouped, False), ("table E=16", other, True),
                         ("table E=8", grouped, True), ("hash E=16", other, False)):
        y_s, y_r = _both(d, lut=lut)
        torch.cuda.synchronize()
        assert not torch.isnan(y_s.float()).any(), name
        assert torch.equal(y_s.view(torch.int16), y_r.view(torch.int16)), name


def test_static_give_up_leaves_later_shapes_exact():
    """A static call of the persistent launch whose waits give up (spin limit
    0, forced from the host: no wait runs, every kernel reaches its end)
    writes NaN and raises the device flag; the next persistent call reports
    it without running.  Later static calls of the two-launch path and of
    another persistent shape then match the workspace entry point
    bit-for-bit: the give-up's status flag is kept outside every shape's
    counters."""
    from escha_mlx_amd import _lib, ops
    k = 8
    ops.init()
    pers = _device(_case(64, 512, 256, 2, k, 913), k)
    two = _device(_case(256, 2048, 512, 1, k, 914), k)
    pers2 = _device(_case(32, 1024, 256, 3, 4, 915), 4)
    y = torch.empty((2, 512), dtype=torch.float16, device=DEV)
    ops.set_moe_spin_limit(0)
    try:
        ops.moe_expert_path_static(*_args(pers), out=y)
        torch.cuda.synchronize()
    finally:
        ops.set_moe_spin_limit(-1)
    assert torch.isnan(y.float()).all()
    with pytest.raises(_lib.EschaWaitTimeout, match="bounded wait"):
        ops.moe_expert_path_static(*_args(pers), out=y)
    for name, d in (("two-launch T=1", two), ("persistent E=32 H=1024 T=3 top-4", pers2),
                    ("persistent T=2", pers), ("two-launch again", two)):
        y_s, y_r = _both(d)
        torch.cuda.synchronize()
        assert not torch.isnan(y_s.float()).any(), name
        assert torch.equal(y_s.view(torch.int16), y_r.view(torch.int16)), name


@pytest.mark.parametrize("shape", ["two-launch", "persistent"])
def test_static_expert_path_in_a_captured_graph(shape):
    """After esc_init, the static call is captured into a HIP graph and
    replayed three times with eager calls of the workspace entry point in
    between: every replay is bit-identical to the eager result."""
    from escha_mlx_amd import ops
    k = 8
    ops.init()
    E, H, I, T = (256, 2048, 512, 1) if shape == "two-launch" else (64, 512, 256, 2)
    d = _device(_case(E, H, I, T, k, 916), k)
    other = _device(_case(E, H, I, T, k, 917), k)
    want = ops.moe_expert_path(*_args(d))
    y_g = torch.empty((T, H), dtype=torch.float16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.moe_expert_path_static(*_args(d), out=y_g)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.moe_expert_path_static(*_args(d), out=y_g)
    for i in range(3):
        y_g.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_g.view(torch.int16), want.view(torch.int16)), f"replay {i}"
        ops.moe_expert_path(*_args(other))
        torch.cuda.synchronize()
