"""GPU: the allocation-free sparse decode entry point
(ekv_sparse_mla_decode_noalloc) through the C ABI against the workspace
entry point (ekv_sparse_mla_decode) on the same inputs: bit-identical out
and lse on two calls in a row, the second smaller; an oversized call is
refused."""

import numpy as np
import pytest
import torch

from helpers import bf16_tensor, randn_bf16, to_dev
from oracle import paged
from oracle.fp8 import quantize_rows

pytestmark = pytest.mark.gpu


def _case(dev, rng, T, H, W, pages=48):
    rows = randn_bf16(rng, (pages * 64, 576))
    pool = np.zeros((pages, paged.fp8_page_bytes(576)), np.uint8)
    c, s = quantize_rows(rows)
    paged.write_fp8_rows(pool, np.arange(pages * 64), c, s, 576)
    idx = rng.integers(0, pages * 64, (T, W)).astype(np.int32)
    idx[:, -7:] = -1
    lengths = rng.integers(0, W + 1, T).astype(np.int32)
    q = randn_bf16(rng, (T, H, 576))
    sinks = rng.standard_normal(H).astype(np.float32)
    return (bf16_tensor(q, dev), to_dev(pool, dev), to_dev(idx, dev), to_dev(lengths, dev), to_dev(sinks, dev))


def _noalloc(q, pool, idx, lengths, sinks, out, lse):
    from ernie_kv import _lib

    T, H, D = q.shape
    _lib.call("ekv_sparse_mla_decode_noalloc", q.data_ptr(), q.stride(0), q.stride(1), T, H, D, pool.data_ptr(), 0,
              pool.stride(0), pool.shape[0], idx.data_ptr(), idx.stride(0), idx.shape[1], lengths.data_ptr(), None, 0,
              None, sinks.data_ptr(), 256 ** -0.5, out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr(),
              lse.stride(0), torch.cuda.current_stream().cuda_stream)


def test_noalloc_decode_matches_workspace_decode(dev):
    from ernie_kv import ops

    rng = np.random.default_rng(91)
    for T, H, W in [(32, 64, 2176), (5, 16, 300)]:  # the second call smaller
        q, pool, idx, lengths, sinks = _case(dev, rng, T, H, W)
        out_ws = torch.full((T, H, 512), 7, dtype=torch.bfloat16, device=dev)
        lse_ws = torch.full((T, H), 7, dtype=torch.float32, device=dev)
        ops.sparse_mla_decode(q, pool, idx, 256 ** -0.5, out_ws, lse_ws, sinks=sinks, lengths=lengths)
        out_na = torch.full((T, H, 512), -7, dtype=torch.bfloat16, device=dev)
        lse_na = torch.full((T, H), -7, dtype=torch.float32, device=dev)
        _noalloc(q, pool, idx, lengths, sinks, out_na, lse_na)
        torch.cuda.synchronize()
        assert torch.equal(out_na.view(torch.int16), out_ws.view(torch.int16)), f"out differs at {(T, H, W)}"
        assert torch.equal(lse_na.view(torch.int32), lse_ws.view(torch.int32)), f"lse differs at {(T, H, W)}"


def test_noalloc_decode_refuses_oversized_calls(dev):
    from ernie_kv import _lib

    lib = _lib.load()
    T, H, W = 1024, 64, 2176
    assert lib.ekv_sparse_mla_decode_workspace_size(T, H, W) > (64 << 20)
    q = torch.zeros((T, H, 576), dtype=torch.bfloat16, device=dev)
    pool = torch.zeros((1, paged.fp8_page_bytes(576)), dtype=torch.uint8, device=dev)
    idx = torch.zeros((T, W), dtype=torch.int32, device=dev)
    lengths = torch.zeros(T, dtype=torch.int32, device=dev)
    sinks = torch.zeros(H, dtype=torch.float32, device=dev)
    out = torch.zeros((T, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.zeros((T, H), dtype=torch.float32, device=dev)
    with pytest.raises(_lib.EkvError, match="more scratch"):
        _noalloc(q, pool, idx, lengths, sinks, out, lse)


def test_noalloc_decode_under_graph_capture(dev):
    """The allocation-free decode captured in a HIP graph (its scratch
    address looked up before capture, on the warm-up call) and replayed three
    times after q and the row lengths are rewritten in place: every replay's
    out and lse equal the workspace entry point's on the same inputs, bit for
    bit, with eager work and synchronizations between the replays."""
    from ernie_kv import ops

    rng = np.random.default_rng(92)
    T, H, W = 16, 64, 1200
    q, pool, idx, lengths, sinks = _case(dev, rng, T, H, W)
    out = torch.zeros((T, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.zeros((T, H), dtype=torch.float32, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _noalloc(q, pool, idx, lengths, sinks, out, lse)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _noalloc(q, pool, idx, lengths, sinks, out, lse)
    torch.cuda.synchronize()
    for rep in range(3):
        q.copy_(bf16_tensor(randn_bf16(rng, (T, H, 576)), dev))
        lengths.copy_(to_dev(rng.integers(0, W + 1, T).astype(np.int32), dev))
        out_ws = torch.full((T, H, 512), 7, dtype=torch.bfloat16, device=dev)
        lse_ws = torch.full((T, H), 7, dtype=torch.float32, device=dev)
        ops.sparse_mla_decode(q, pool, idx, 256 ** -0.5, out_ws, lse_ws, sinks=sinks, lengths=lengths)
        out.fill_(0)
        lse.fill_(0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), out_ws.view(torch.int16)), f"replay {rep}: out"
        assert torch.equal(lse.view(torch.int32), lse_ws.view(torch.int32)), f"replay {rep}: lse"
