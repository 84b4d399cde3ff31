"""The loss steps captured in a HIP graph and replayed.

A small batch is launch-bound: at c1's shape (fp32 [4, 256, 32000]) the
kernels take a fraction of the step's wall time. A caller can capture the
whole forward + backward with ``torch.cuda.graph`` (target validation off:
its host wait cannot be captured) and replay it on new data copied into the
static inputs. Each replay must give exactly the eager result on the same
data (the kernels are deterministic), with eager work and synchronisations
between the replays. The fused LM head + loss is captured the same way; its
backward's library GEMMs run inside the graph too. The one-pass path is
captured with a scaled loss as well: the upstream value its forward assumes
comes from a device tensor that the backward writes, so replays keep the
forward's gradient.
"""

from __future__ import annotations

import time

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _capture(step, warmup=2):
    """Warm ``step`` up on a side stream, then capture it; returns the graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    return graph, out


def test_unfused_step_replays_exactly():
    import nmce
    ctx = nmce.ParallelContext.single()
    b, s, v = 4, 256, 32000
    logits = torch.zeros(b, s, v, device=DEV, requires_grad=True)
    target = torch.zeros(b, s, dtype=torch.int64, device=DEV)

    def step():
        logits.grad = None
        loss = nmce.vocab_parallel_cross_entropy(logits, target, 0, v, ctx, validate=False)
        loss.backward()
        return loss.detach()  # keep no autograd graph alive between steps

    graph, static_loss = _capture(step)
    g = torch.Generator().manual_seed(3)
    for rep in range(4):
        x = torch.randn(b, s, v, generator=g) * 2.0
        t = torch.randint(0, v, (b, s), generator=g)
        with torch.no_grad():
            logits.copy_(x.to(DEV))
        target.copy_(t.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got_loss, got_grad = static_loss.item(), logits.grad.clone()
        # eager on the same data, with its own allocations and host checks
        xe = x.to(DEV).requires_grad_(True)
        le = nmce.vocab_parallel_cross_entropy(xe, t.to(DEV), 0, v, ctx)
        le.backward()
        torch.cuda.synchronize()
        assert got_loss == le.item(), f"replay {rep}: loss {got_loss} vs eager {le.item()}"
        assert torch.equal(got_grad, xe.grad), f"replay {rep}: gradient differs from eager"

    # launch-bound: report what the replay saves (informational)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(50):
        graph.replay()
    torch.cuda.synchronize()
    t_graph = (time.perf_counter() - t0) / 50
    t0 = time.perf_counter()
    for _ in range(50):
        step()
    torch.cuda.synchronize()
    t_eager = (time.perf_counter() - t0) / 50
    print(f"[graph] c1 step: eager {t_eager * 1e3:.3f} ms, replay {t_graph * 1e3:.3f} ms",
          flush=True)


def test_fused_step_replays_exactly():
    import nmce
    ctx = nmce.ParallelContext.single()
    n, h, v = 512, 256, 5000
    hidden = torch.zeros(n, h, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    weight = torch.zeros(v, h, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    target = torch.zeros(n, dtype=torch.int64, device=DEV)

    def step():
        hidden.grad = None
        weight.grad = None
        loss = nmce.lmhead_vocab_parallel_cross_entropy(hidden, weight, target, 0, v, ctx,
                                                        vocab_chunk=2048, validate=False)
        loss.backward()
        return loss.detach()

    graph, static_loss = _capture(step)
    g = torch.Generator().manual_seed(4)
    for rep in range(4):
        x = torch.randn(n, h, generator=g).to(torch.bfloat16)
        w = (torch.randn(v, h, generator=g) * 0.3).to(torch.bfloat16)
        t = torch.randint(0, v, (n,), generator=g)
        with torch.no_grad():
            hidden.copy_(x.to(DEV))
            weight.copy_(w.to(DEV))
        target.copy_(t.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got = (static_loss.item(), hidden.grad.clone(), weight.grad.clone())
        xe = x.to(DEV).requires_grad_(True)
        we = w.to(DEV).requires_grad_(True)
        le = nmce.lmhead_vocab_parallel_cross_entropy(xe, we, t.to(DEV), 0, v, ctx,
                                                      vocab_chunk=2048)
        le.backward()
        torch.cuda.synchronize()
        assert got[0] == le.item(), f"replay {rep}: loss {got[0]} vs eager {le.item()}"
        assert torch.equal(got[1], xe.grad), f"replay {rep}: hidden gradient differs"
        assert torch.equal(got[2], we.grad), f"replay {rep}: weight gradient differs"


def test_one_pass_scaled_loss_replays_exactly():
    """The one-pass path inside a graph with the loss scaled by 0.5 each step (as
    a pipeline scales by 1/num_microbatches): the upstream value the forward
    assumes comes from a device tensor the backward writes, so replays keep
    the forward's gradient and match eager steps bit for bit."""
    import nmce
    ctx = nmce.ParallelContext.single()
    n, v = 512, 8192
    logits = torch.zeros(n, v, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    target = torch.zeros(n, dtype=torch.int64, device=DEV)

    def step():
        logits.grad = None
        loss = nmce.vocab_parallel_cross_entropy(logits, target, 0, v, ctx, validate=False)
        (loss * 0.5).backward()
        return loss.detach()

    graph, static_loss = _capture(step)
    g = torch.Generator().manual_seed(8)
    for rep in range(3):
        x = (torch.randn(n, v, generator=g) * 2.0).to(torch.bfloat16)
        t = torch.randint(0, v, (n,), generator=g)
        with torch.no_grad():
            logits.copy_(x.to(DEV))
        target.copy_(t.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got = (static_loss.item(), logits.grad.clone())
        xe = x.to(DEV).requires_grad_(True)
        le = nmce.vocab_parallel_cross_entropy(xe, t.to(DEV), 0, v, ctx, one_pass=False)
        (le * 0.5).backward()
        torch.cuda.synchronize()
        assert got[0] == le.item(), f"replay {rep}: loss {got[0]} vs eager {le.item()}"
        assert torch.equal(got[1].view(torch.int16), xe.grad.view(torch.int16)), \
            f"replay {rep}: gradient differs from the two-pass eager step"
