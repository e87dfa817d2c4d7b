"""CPU regression test of the decode graph's body (nanopd_amd/graphs.py).

A captured copy_ between device tensors becomes a memcpy node of the HIP
graph. An earlier body ended with tokens.copy_(logits.argmax(-1)): a memcpy
node whose source, the argmax result, was an intermediate in the memory pool
that every decode graph shares, where other graphs keep bf16 activations. A
replay whose copy read that address before argmax had written it would hand
the engine another graph's bf16 bits as a token id (what a served FP8 run
once stopped on). The body now has argmax write the token buffer itself
(argmax(..., out=tokens)), so the graph holds kernel nodes only; the GPU test
tests/test_gpu_graphs.py::test_decode_graph_holds_kernel_nodes_only lists
the captured nodes. Here the body runs on CPU tensors with a stub model under
a dispatch mode that records every aten op."""
import types

import torch
from torch.utils._python_dispatch import TorchDispatchMode

from nanopd_amd import _lib, graphs


class _Record(TorchDispatchMode):
    def __init__(self):
        super().__init__()
        self.ops = []

    def __torch_dispatch__(self, func, types_, args=(), kwargs=None):
        kwargs = kwargs or {}
        out = kwargs.get("out")
        self.ops.append((func, out.data_ptr() if isinstance(out, torch.Tensor) else None))
        return func(*args, **kwargs)


class _StubModel:
    def __init__(self, vocab: int):
        self.device = torch.device("cpu")
        self.block_size = 16
        self.vocab = vocab
        self.batches = []

    def forward(self, batch):
        self.batches.append(batch)
        n = batch.input_ids.numel()
        g = torch.Generator().manual_seed(n)
        return torch.randn(n, self.vocab, generator=g).to(torch.bfloat16)


def _body_graph(monkeypatch, batch=4, width=16, vocab=1000):
    monkeypatch.setattr(_lib, "call", lambda *a, **k: None)
    monkeypatch.setattr(torch.cuda, "current_stream",
                        lambda dev=None: types.SimpleNamespace(cuda_stream=0))
    g = object.__new__(graphs._Graph)
    g.batch, g.width = batch, width
    g.model = _StubModel(vocab)
    g.staging = torch.zeros(batch + 3 * batch + batch * width, dtype=torch.int32)
    out = torch.zeros(batch + 1 + batch + batch * width + 3 * batch, dtype=torch.int32)
    o = 0
    g.cu = out[o:o + batch + 1]; o += batch + 1
    g.seq_lens = out[o:o + batch]; o += batch
    g.tables = out[o:o + batch * width].view(batch, width); o += batch * width
    g.positions = out[o:o + batch]; o += batch
    g.slots = out[o:o + batch]; o += batch
    g.token_seq = out[o:o + batch]
    g.workspace = torch.zeros(64, dtype=torch.uint8)
    g.tokens = torch.full((batch,), -1, dtype=torch.int64)
    return g


def test_graph_body_writes_tokens_with_argmax_out_and_no_copy(monkeypatch):
    g = _body_graph(monkeypatch)
    rec = _Record()
    with rec:
        g._body()
    names = [str(f) for f, _ in rec.ops]
    assert not [n for n in names if n.startswith("aten.copy_")], names
    writes = [n for (f, ptr), n in zip(rec.ops, names) if ptr == g.tokens.data_ptr()]
    assert writes == ["aten.argmax.out"], names
    want = g.model.forward(g.model.batches[0]).float().argmax(-1)
    assert torch.equal(g.tokens, want)
    assert g.model.batches[0].decode_workspace is g.workspace


def test_planted_copy_into_tokens_is_caught(monkeypatch):
    """The earlier body (argmax into a temporary, then copy_) fails the check
    above: the recorder sees the copy_."""
    g = _body_graph(monkeypatch)
    real = torch.argmax

    def old_style(x, dim=None, out=None, **kw):
        assert out is g.tokens
        return out.copy_(real(x, dim=dim))

    monkeypatch.setattr(torch, "argmax", old_style)
    rec = _Record()
    with rec:
        g._body()
    assert any(str(f).startswith("aten.copy_") for f, _ in rec.ops)
