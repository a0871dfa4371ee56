"""The decode chain (fp8lin_decode_chain): the one-row projections of a decode
step in one launch, each link waiting for the link whose output it
reads (Engine::step's linear calls at one token, src/engine.cpp:401-421).

Every link's output must equal the same projection through fp8_linear
(linear_swiglu for SwiGLU links) bit for bit -- the chain sums each row in the
decode GEMV's order -- and those per-link calls are held to the FP64 oracle
here as well.  After every call no wait may have given up (sync word 0 stays
zero) and every link counter must have advanced by the link's number of
workgroups at every call.
"""
import numpy as np
import pytest
import torch

from parity import assert_parity

pytestmark = pytest.mark.gpu


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def link_workgroups(link):
    """Workgroups of a chain link: 8 items each (4 waves of 2 items), an
    item 2 rows (a gate/up pair with SwiGLU) for K <= 5120, else 1 row."""
    codes, swiglu = link[1], bool(link[3]) if len(link) > 3 else False
    n, k = codes.shape
    items = n // 2 if swiglu else ((n + 1) // 2 if k <= 5120 else n)
    return -(-items // 8)


def check_sync(ws, links, calls):
    """Word 0 (waits that gave up) is zero, word 1 holds the chain's
    signature; the 256 slot counters of each link
    that waits or is waited for (one per 128-byte line from word 16) sum to
    calls x the link's workgroup count, the others stay zero; the per-XCD
    words of a link that waits (one per 256 bytes after
    the counters) hold the last call index + 1 where set, and nothing else
    is touched."""
    n = len(links)
    w = ws.view(torch.int64).cpu().numpy()
    assert w[0] == 0, w[:16]
    assert w[1] != 0 and not w[2:16].any(), w[:16]  # the chain's signature
    cnt = w[16:16 + n * 256 * 16].reshape(n, 256, 16)
    assert not cnt[:, :, 1:].any()
    def after(link):
        return link[4] if len(link) > 4 and link[4] is not None else (link[0] if isinstance(link[0], int) else -1)
    waited = {after(link) for link in links}
    for i, link in enumerate(links):
        counted = i in waited or after(link) >= 0  # links waited for, or waiting
        assert cnt[i, :, 0].sum() == (calls * link_workgroups(link) if counted else 0), (i, cnt[i, :, 0].sum())
    xw = w[16 + n * 256 * 16:16 + n * 256 * 16 + n * 8 * 32].reshape(n, 8, 32)
    assert not xw[:, :, 1:].any()
    for i, link in enumerate(links):
        if after(link) >= 0:
            assert xw[i, :, 0].max() == calls and xw[i, :, 0].min() >= 0, xw[i, :, 0]
        else:
            assert not xw[i, :, 0].any(), xw[i, :, 0]
    assert not w[16 + n * 256 * 16 + n * 8 * 32:].any()


def per_link(F, links, outs):
    """The same links through the single-projection operators."""
    want = []
    for x, codes, scales, *rest in links:
        swiglu = bool(rest[0]) if rest else False
        xx = outs[x] if isinstance(x, int) else x
        want.append(F.linear_swiglu(xx, codes, scales) if swiglu else F.fp8_linear(xx, codes, scales, True))
    return want


def test_chain_layer_and_head(fp8lin, gpu, oracle):
    """BASELINE config 5 at decode: QKV-gate 7168x5120 -> gate/up + SwiGLU
    17408x5120 -> down 5120x8704 -> vocab-sharded head 75968x5120, each link
    after the previous one (gate/up reads the layer input, as the benchmark's
    chain does, but waits for QKV-gate as it waits for attention in a layer),
    twice on one workspace."""
    F = fp8lin
    shapes = [(7168, 5120), (17408, 5120), (5120, 8704), (75968, 5120)]
    w = [F.gen_weights(n, k, seed=0, tag=60 + i, device=gpu) for i, (n, k) in enumerate(shapes)]
    ws = F.decode_chain_workspace(4, gpu)
    for rep in range(2):
        x = F.gen_activations(1, 5120, seed=rep, tag=66, device=gpu)
        links = [(x, *w[0]), (x, *w[1], True, 0), (1, *w[2]), (2, *w[3])]
        outs = F.decode_chain(links, ws)
        torch.cuda.synchronize()
        check_sync(ws, links, rep + 1)
        for i, (got, want) in enumerate(zip(outs, per_link(F, links, outs))):
            assert torch.equal(got, want), f"link {i} rep {rep}"
    xb = bits(x)
    assert_parity(bits(outs[0]), oracle.linear(xb, w[0][0].cpu().numpy(), w[0][1].cpu().numpy()), "chain QKV-gate")
    ref_gu = oracle.linear(xb, w[1][0].cpu().numpy(), w[1][1].cpu().numpy())
    assert_parity(bits(outs[1]), oracle.swiglu(ref_gu), "chain gate/up+SwiGLU", elementwise=False)
    assert_parity(bits(outs[2]), oracle.linear(bits(outs[1]), w[2][0].cpu().numpy(), w[2][1].cpu().numpy()),
                  "chain down")
    assert_parity(bits(outs[3]), oracle.linear(bits(outs[2]), w[3][0].cpu().numpy(), w[3][1].cpu().numpy()),
                  "chain head")


def rand_case(rng, gpu, n, k, per_row=False):
    codes = rng.integers(0, 127, (n, k), dtype=np.uint8) | (rng.integers(0, 2, (n, k), dtype=np.uint8) << 7)
    cols = 1 if per_row else (k + 127) // 128
    scales = (rng.random((n, cols)) * .01 + .001).astype(np.float32)
    if per_row:
        scales = scales[:, 0].copy()
    return torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu)


def rand_x(rng, gpu, k, scale=1.0):
    f = (rng.standard_normal((1, k)) * scale).astype(np.float32)
    return torch.from_numpy(f).to(torch.bfloat16).to(gpu)


def test_chain_shapes(fp8lin, gpu, oracle):
    """Every item form and edge in one chain of 8 links: K not a multiple of
    1024 (4112: a partial last step; 1008), 9 full steps (9216), per-row
    scales, an odd number of rows (1001: a last pair with one row), a SwiGLU
    link with an odd number of pairs (1025), links with fewer items than the
    grid has waves (48 and 3 rows: most waves own none), K = 16 (one chunk),
    waits on links other than the previous one, and a link that reads the
    previous link's output."""
    F = fp8lin
    rng = np.random.default_rng(61)
    spec = [  # (N, K, per-row scales)
        (1001, 4112, True), (2050, 1024, False), (300, 9216, False), (48, 1008, False),
        (3, 1024, False), (4096, 16, False), (640, 1024, False), (512, 640, False)]
    w = [rand_case(rng, gpu, n, k, pr) for n, k, pr in spec]
    xs = {i: rand_x(rng, gpu, spec[i][1]) for i in (0, 1, 2, 3, 5, 6)}
    links = [(xs[0], *w[0]), (xs[1], *w[1], True), (xs[2], *w[2], False, 1), (xs[3], *w[3], False, 0),
             (xs[1], *w[4], False, -1), (xs[5], *w[5], False, 3), (xs[6], *w[6]), (6, *w[7])]
    ws = F.decode_chain_workspace(8, gpu)
    outs = F.decode_chain(links, ws)
    torch.cuda.synchronize()
    check_sync(ws, links, 1)
    for i, (got, want) in enumerate(zip(outs, per_link(F, links, outs))):
        assert torch.equal(got, want), f"link {i}"
    assert_parity(bits(outs[0]), oracle.linear(bits(xs[0]), w[0][0].cpu().numpy(), w[0][1].cpu().numpy()),
                  "chain K=4112 per-row scales")
    assert_parity(bits(outs[2]), oracle.linear(bits(xs[2]), w[2][0].cpu().numpy(), w[2][1].cpu().numpy()),
                  "chain K=9216")
    assert_parity(bits(outs[7]), oracle.linear(bits(outs[6]), w[7][0].cpu().numpy(), w[7][1].cpu().numpy()),
                  "chain link fed by the previous one")


def test_chain_graph_replay(fp8lin, gpu):
    """The chain captured in a HIP graph and replayed with new activations,
    eager work and synchronisations in between: each replay equals the
    per-link operators on the same input and advances every link counter by
    its workgroup count, with no wait given up."""
    F = fp8lin
    shapes = [(7168, 5120), (17408, 5120), (5120, 8704)]
    w = [F.gen_weights(n, k, seed=1, tag=70 + i, device=gpu) for i, (n, k) in enumerate(shapes)]
    x = F.gen_activations(1, 5120, seed=0, tag=76, device=gpu)
    links = [(x, *w[0]), (x, *w[1], True, 0), (1, *w[2])]
    ws = F.decode_chain_workspace(3, gpu)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        F.decode_chain(links, ws)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            outs = F.decode_chain(links, ws)
    for i in range(3):
        x.copy_(F.gen_activations(1, 5120, seed=10 + i, tag=76, device=gpu))
        F.fp8_linear(x, *w[0])  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        check_sync(ws, links, i + 2)
        for j, (got, want) in enumerate(zip(outs, per_link(F, links, outs))):
            assert torch.equal(got, want), f"replay {i} link {j}"


def test_chain_workspace_of_another_chain(fp8lin, gpu):
    """A workspace that counted one chain, then given a chain of another
    shape, makes every wait of the new chain give up at once (each counted
    in word 0) rather than wait for counts that never come; zeroed, it serves
    the new chain.  Small links, so that all workgroups are resident."""
    F = fp8lin
    rng = np.random.default_rng(62)
    a = [rand_case(rng, gpu, n, 1024) for n in (512, 256)]
    b = [rand_case(rng, gpu, n, 1024) for n in (1024, 256)]
    x = rand_x(rng, gpu, 1024)
    first = [(x, *a[0]), (x, *a[1], False, 0)]
    second = [(x, *b[0]), (x, *b[1], False, 0)]
    ws = F.decode_chain_workspace(2, gpu)
    F.decode_chain(first, ws)
    torch.cuda.synchronize()
    check_sync(ws, first, 1)
    sig = int(ws.view(torch.int64)[1])
    F.decode_chain(second, ws)
    torch.cuda.synchronize()
    w = ws.view(torch.int64).cpu()
    assert int(w[0]) == link_workgroups(second[1]), int(w[0])  # every waiting workgroup gave up
    assert int(w[1]) == sig  # the first chain's signature stays
    ws.zero_()
    outs = F.decode_chain(second, ws)
    torch.cuda.synchronize()
    check_sync(ws, second, 1)
    for i, (got, want) in enumerate(zip(outs, per_link(F, second, outs))):
        assert torch.equal(got, want), f"link {i}"
