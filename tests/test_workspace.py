"""Workspace pool: per-stream buffers that only grow, and replaced buffers kept alive for captured graphs.

Runs on the CPU: the stream lookup is stubbed and the buffers are host tensors (the pool's bookkeeping does not
depend on where they live).
"""

import types

import torch

from aicas_amd import ops


def _stub_streams(monkeypatch, stream_id):
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device=None: types.SimpleNamespace(cuda_stream=stream_id[0]))


def test_grows_and_keeps_replaced_buffers_alive(monkeypatch):
    stream = [11]
    _stub_streams(monkeypatch, stream)
    ops.Workspace.clear()
    try:
        dev = torch.device("cpu")
        a = ops.Workspace.get(dev, 1000)
        assert a.numel() >= 1 << 20 and int(a.sum()) == 0
        assert ops.Workspace.get(dev, 4096).data_ptr() == a.data_ptr()  # reused while large enough
        b = ops.Workspace.get(dev, (3 << 20) + 5)
        assert b.numel() >= (3 << 20) + 5 and b.data_ptr() != a.data_ptr() and int(b.sum()) == 0
        # the replaced buffer is still referenced by the pool: a graph captured on it stays valid
        assert any(r.data_ptr() == a.data_ptr() for r in ops.Workspace._retired)
        # another stream gets its own buffer
        stream[0] = 12
        c = ops.Workspace.get(dev, 1000)
        assert c.data_ptr() not in (a.data_ptr(), b.data_ptr())
        stream[0] = 11
        assert ops.Workspace.get(dev, 1000).data_ptr() == b.data_ptr()
    finally:
        ops.Workspace.clear()
    assert not ops.Workspace._pool and not ops.Workspace._retired
