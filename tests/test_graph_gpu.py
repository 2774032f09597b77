"""The C-ABI entry points under HIP graph capture (torch.cuda.graph): a
captured vcpp_paged_decode, vcpp_paged_prefill_split and
vcpp_paged_mixed_step (whose decode merge forks onto a side stream and joins
back by events) replay bit-identically to the eager calls, three replays in
a row with eager work on the outputs between them.  The kernels' split and
merge orders are fixed by the shapes, so eager and replayed results are
bit-equal."""
import pytest
import torch

import pyvcpp

pytestmark = pytest.mark.gpu

BS, HKV, D, H = 16, 8, 80, 64


def setup(seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    dev = torch.device("cuda:0")
    dctx = torch.randint(1, 3000, (24,), generator=g, dtype=torch.int32)
    prefix = [2500, 0, 700]
    chunk = [64, 130, 1]
    lens = dctx.tolist() + [p + c for p, c in zip(prefix, chunk)]
    nblk = [(n + BS - 1) // BS for n in lens]
    nb = sum(nblk) + 8
    k = torch.randn((nb, BS, HKV, D), generator=g).half().to(dev)
    v = torch.randn((nb, BS, HKV, D), generator=g).half().to(dev)
    pages = pyvcpp.kv_pages(pyvcpp.KV_F16, k, v, BS, HKV, D, nb, BS * HKV * D)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    tab = torch.full((len(lens), max(nblk)), -1, dtype=torch.int32)
    o = 0
    for i, n in enumerate(nblk):
        tab[i, :n] = perm[o:o + n]
        o += n
    w = dict(pages=pages, k=k, v=v,
             dtab=tab[:24].contiguous().to(dev), ptab=tab[24:].contiguous().to(dev),
             dctx=dctx.to(dev), max_ctx=int(dctx.max()),
             dq=torch.randn((24, H, D), generator=g).to(dev),
             pq=torch.randn((sum(chunk), H, D), generator=g).half().view(torch.int16).to(dev),
             q_start=torch.tensor([0, 64, 194, 195], dtype=torch.int32, device=dev),
             prefix=torch.tensor(prefix, dtype=torch.int32, device=dev), max_chunk=max(chunk),
             max_prefix=max(prefix))
    w["dout"] = torch.empty_like(w["dq"])
    w["pout"] = torch.empty((sum(chunk), H, D), dtype=torch.float32, device=dev)
    return w


def decode(w, ws):
    pyvcpp.paged_decode(w["pages"], w["dq"], w["dout"], w["dtab"], w["dctx"], w["max_ctx"], H, workspace=ws)


def prefill_split(w, ws):
    pyvcpp.paged_prefill_split(w["pages"], w["pq"], w["pout"], w["ptab"], w["q_start"], w["prefix"],
                               w["max_chunk"], w["max_prefix"], H, workspace=ws)


def mixed(w, ws):
    pyvcpp.paged_mixed_step(w["pages"], w["dq"], w["dout"], w["dtab"], w["dctx"], w["max_ctx"], w["pq"],
                            w["pout"], w["ptab"], w["q_start"], w["prefix"], w["max_chunk"], H, workspace=ws)


def workspace(w, which):
    p = w["pages"]
    if which == "decode":
        n = pyvcpp.decode_workspace_size(p, 24, H, w["max_ctx"], 0)
    elif which == "prefill_split":
        n = pyvcpp.prefill_workspace_size(p, 3, w["max_chunk"], w["max_prefix"], H)
    else:
        n = pyvcpp.mixed_workspace_size(p, 24, H, w["max_ctx"], w["ptab"].shape[1])
    return torch.zeros(max(n, 1), dtype=torch.uint8, device="cuda:0")


@pytest.mark.parametrize("which", ["decode", "prefill_split", "mixed"])
def test_graph_replays_match_eager(cuda, which):
    w = setup(90 + len(which))
    fn = {"decode": decode, "prefill_split": prefill_split, "mixed": mixed}[which]
    outs = {"decode": ["dout"], "prefill_split": ["pout"], "mixed": ["dout", "pout"]}[which]
    ws = workspace(w, which)
    if which == "prefill_split":
        assert ws.numel() > 1, "shape was meant to split"
    fn(w, ws)
    torch.cuda.synchronize()
    ref = {o: w[o].clone() for o in outs}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(w, ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn(w, ws)
    torch.cuda.synchronize()
    for rep in range(3):
        for o in outs:
            w[o].fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o in outs:
            assert torch.equal(w[o], ref[o]), "%s: replay %d of %s differs from the eager call" % (which, rep, o)


def test_mixed_capture_beside_eager_stream(cuda):
    """One stream captures a mixed step while another stream of the same GPU
    runs mixed steps eagerly inside the capture: each caller stream forks its
    merge onto its own side stream, so the eager steps are neither recorded
    into the graph nor break the capture, and both results match the eager
    reference (the graph over three replays)."""
    wa = setup(97)
    wb = setup(98)
    wsa = workspace(wa, "mixed")
    wsb = workspace(wb, "mixed")
    mixed(wa, wsa)
    mixed(wb, wsb)
    torch.cuda.synchronize()
    ref_a = {o: wa[o].clone() for o in ("dout", "pout")}
    ref_b = {o: wb[o].clone() for o in ("dout", "pout")}
    sb = torch.cuda.Stream()
    sb.wait_stream(torch.cuda.current_stream())

    def mixed_b():
        pyvcpp.paged_mixed_step(wb["pages"], wb["dq"], wb["dout"], wb["dtab"], wb["dctx"], wb["max_ctx"], wb["pq"],
                                wb["pout"], wb["ptab"], wb["q_start"], wb["prefix"], wb["max_chunk"], H,
                                workspace=wsb, stream=sb)

    mixed_b()  # its side stream exists before the capture
    torch.cuda.synchronize()
    for o in ("dout", "pout"):
        wb[o].fill_(float("nan"))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        mixed(wa, wsa)
        mixed_b()  # eager, on stream sb, while the capture is open
        mixed(wa, wsa)
    torch.cuda.synchronize()
    for o in ("dout", "pout"):
        assert torch.equal(wb[o], ref_b[o]), "eager step beside the capture: %s differs" % o
    for rep in range(3):
        for o in ("dout", "pout"):
            wa[o].fill_(float("nan"))
            wb[o].fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o in ("dout", "pout"):
            assert torch.equal(wa[o], ref_a[o]), "replay %d: %s differs" % (rep, o)
            # nothing of stream b's step was recorded into the graph
            assert torch.isnan(wb[o]).all(), "replay %d wrote stream b's %s" % (rep, o)
