"""Broadcast products (the product kernel's outer-axis path, configs 4b and
5.R) at sizes where every thread of the grid runs several grid-stride
iterations (MI355X: 256 CUs x 64 blocks x 256 threads): the software-
pipelined main loop (next iteration's loads before this iteration's stores,
two register sets in turn, entered after an odd or even number of
iterations) and the checked tail that follows it, bit-exact against the
oracle (the reference's elementwise path, pto_einsum_elementwise.h:152-370:
+0 plus the float32 product)."""
import pytest
import torch

import oracle
from parity_util import check

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("eq,s0,s1,dt", [
    ("bsd,d->bsd", (4, 4201, 4096), (4096,), torch.float16),      # 8-wide vectors, ~2.05 iterations
    ("bsd,d->bsd", (3, 4201, 4096), (4096,), torch.float32),      # 4-wide, ~3.1 iterations
    ("bshd,sd->bshd", (6, 4099, 16, 128), (4099, 128), torch.float32),
    ("ij,i->ij", (25003, 2048), (25003,), torch.float32),        # B broadcast along rows
])
def test_broadcast_stream_several_iterations(eq, s0, s1, dt):
    from pto_einsum import einsum

    print(f"product stream: {eq} {s0} x {s1} {dt}", flush=True)
    g = torch.Generator().manual_seed(sum(s0) + len(eq))
    x = torch.randn(s0, generator=g).to(dt)
    y = (torch.rand(s1, generator=g) + 0.5).to(dt)
    got = einsum(eq, x.cuda(), y.cuda()).cpu().numpy()
    want = oracle.einsum(eq, x.float().numpy(), y.float().numpy())
    check(got, want, True, 0, eq)
