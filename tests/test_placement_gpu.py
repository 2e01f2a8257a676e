"""GPU: the restickifies a placement plan lists run through the relayout
kernels (``restickify``) and give the oracle's bytes for the target layout
(bit-exact)."""

import numpy as np
import pytest
import torch

from oracle import layout as OL
from oracle import relayout as OR
from tests.conftest import SEED
from tests.test_placement import GRAPHS, build

pytestmark = pytest.mark.gpu


def _order(layout):
    n = len(layout.size)
    if layout.stick < 0:
        return list(range(n)) + [-1]
    return [d for d in range(n) if d != layout.stick] + [layout.stick]


@pytest.mark.parametrize("name", ["adds_then_matmul_x", "matmul_both_inputs_upstream_conflict",
                                  "4d_mixed_conflicts", "chain_transposed_intermediate"])
def test_planned_restickifies_run_on_gpu(cuda, name):
    import torch_spyre_amd as tsa
    from torch_spyre_amd import placement as RP

    plan = RP.optimize_restickify_locations(build(name))
    sched = RP.schedule(plan)
    assert sched and RP.plan_cost(plan) == GRAPHS[name][1]
    for i, (op, buf, src, dst) in enumerate(sched):
        entry = next(e for e in plan[op] if e["input"] == buf)
        size = list(entry["target_layout"].size)
        strides = OL.contiguous_strides(size)
        bits = OR.random_finite_f16_bits((int(np.prod(size)),), SEED + i)
        x = torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.float16).view(size)
        dev = tsa.to_device_layout(x, src)
        out = tsa.restickify(dev, dst)
        o = OL.stl_init(size, strides, "float16", _order(entry["target_layout"]))
        assert (list(dst.device_size), list(dst.stride_map)) == (o.device_size, o.stride_map)
        want = OL.h2d(bits, size, strides, 0, o)
        got = tsa.device_buffer(out).contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
        assert np.array_equal(got[: want.size], want), (name, op, buf)
