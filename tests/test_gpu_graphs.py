"""Decode-only engine steps replayed from HIP graphs (nanopd_amd/graphs.py)
against the same steps launched kernel by kernel: the graph runs the same
kernels with the same arguments, so for the same padded batch the greedy
tokens are identical. Replays are checked several times, with eager work and
synchronisations between them (a graph that recorded a memset or kept a
stale buffer would diverge after the first replay)."""
import pytest
import torch

from nanopd_amd import paged_kernels as pk
from nanopd_amd.engine import Engine, Request, make_requests
from nanopd_amd.graphs import DecodeGraphs
from nanopd_amd.qwen3 import PagedQwen3, StepBatch
from nanopd_amd.qwen3 import Qwen3Config

SMALL = Qwen3Config(num_layers=3, hidden=1024, num_heads=16, num_kv_heads=4, head_dim=128,
                    intermediate=2048, vocab=4096, init_std=0.05)

pytestmark = pytest.mark.gpu


def _model(device):
    return PagedQwen3(SMALL, num_blocks=512, block_size=16, device=device, seed=3)


def _eager_tokens(model, positions, tables, last, batch, width):
    """The graph's padded step, launched op by op."""
    n = len(positions)
    seqs = [(1, p, t) for p, t in zip(positions, tables)]
    seqs += [(1, -1, [])] * (batch - n)
    meta = pk.pack_metadata(seqs, model.block_size, model.device, max_blocks_per_seq=width)
    ids = torch.tensor(list(last) + [0] * (batch - n), dtype=torch.int64, device=model.device)
    ws = torch.zeros(pk.attention_workspace_bytes(batch, SMALL.num_heads, SMALL.num_kv_heads,
                                                  SMALL.head_dim, model.block_size, width),
                     dtype=torch.uint8, device=model.device)
    b = StepBatch(input_ids=ids, meta=meta, num_prefill_seqs=0, num_prefill_tokens=0,
                  sample_rows=None, decode_workspace=ws)
    return model.forward(b).argmax(-1)[:n].tolist()


def _prefilled(device, n, seed):
    """An engine whose n sequences have finished their prefill."""
    model = _model(device)
    eng = Engine(model, max_batch_size=16, budget=512, chunk=256)
    reqs = make_requests(n, seed=seed, prompt_median=120, prompt_clip=(20, 400), out_median=40,
                         out_clip=(30, 60), vocab=SMALL.vocab)
    for r in reqs:
        eng.add(Request(r.rid, list(r.prompt), r.max_new_tokens))
    while eng.sched.waiting or eng.sched.prefilling:
        eng.step()
    return model, eng


def test_graph_step_equals_eager_step(device):
    model, eng = _prefilled(device, 5, seed=4)
    graphs = DecodeGraphs(model, max_width=64)
    for rep in range(3):
        plan = eng.sched.schedule(0.0)
        assert plan.prefill is None and len(plan.decodes) == 5
        _, seqs, ids, _, _ = eng._rows(plan)
        pos = [c for _, c, _ in seqs]
        tabs = [t for _, _, t in seqs]
        width = max(len(t) for t in tabs)
        g = graphs.capture(len(pos), width)
        assert g.batch == 8 and width <= g.width < 2 * width and g.width & (g.width - 1) == 0
        got = graphs.decode(pos, tabs, ids)
        torch.cuda.synchronize()
        want = _eager_tokens(model, pos, tabs, ids, g.batch, g.width)   # eager work between replays
        assert got == want, f"replay {rep}: {got} != {want}"
        eng.commit(plan, got)


def test_engine_with_graphs_matches_eager_engine(device):
    """Two identical engines serve the same requests, one replaying decode
    steps from graphs. Their GEMMs see different row counts (padded batch),
    so rare argmax flips are allowed; every request must finish."""
    reqs = make_requests(7, seed=9, prompt_median=100, prompt_clip=(20, 300), out_median=20,
                         out_clip=(10, 30), vocab=SMALL.vocab)
    outs = []
    for use in (False, True):
        model = _model(device)
        eng = Engine(model, max_batch_size=16, budget=512, chunk=256,
                     graphs=DecodeGraphs(model, max_width=64) if use else None)
        seqs = [eng.add(Request(r.rid, list(r.prompt), r.max_new_tokens)) for r in reqs]
        eng.drain()
        assert all(len(s.output) == s.req.max_new_tokens for s in seqs)
        assert eng.blocks.num_free_blocks == 512
        outs.append([tok for s in seqs for tok in s.output])
    same = sum(a == b for a, b in zip(*outs)) / len(outs[0])
    print(f"graph engine agrees on {same:.1%} of {len(outs[0])} tokens")
    assert same >= 0.9


def test_steps_without_a_graph_fall_back(device):
    model, eng = _prefilled(device, 3, seed=6)
    graphs = DecodeGraphs(model, max_width=16)
    assert graphs.bucket(3, 17) is None and graphs.bucket(17, 4) is None
    assert graphs.decode([5], [[1] * 17], [0]) is None
    assert graphs.bucket(3, 5) == (4, 16)



def _node_types(graph_handle: int) -> list:
    """hipGraphNodeType of every node of a captured graph (HIP runtime API)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    n = ctypes.c_size_t(0)
    assert hip.hipGraphGetNodes(ctypes.c_void_p(graph_handle), None, ctypes.byref(n)) == 0
    nodes = (ctypes.c_void_p * n.value)()
    assert hip.hipGraphGetNodes(ctypes.c_void_p(graph_handle), nodes, ctypes.byref(n)) == 0
    types = []
    for i in range(n.value):
        t = ctypes.c_int(-1)
        assert hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(t)) == 0
        types.append(t.value)
    return types


def test_decode_graph_holds_kernel_nodes_only(device):
    """The captured decode step is kernel nodes only: no memcpy node (argmax
    writes the token buffer itself; the staging upload happens before the
    replay) and no memset node."""
    from nanopd_amd.graphs import _Graph
    model = _model(device)
    g = _Graph(model, 4, 32, debug=True)
    types = _node_types(g.graph.raw_cuda_graph())
    kinds = {t: types.count(t) for t in set(types)}
    print(f"decode graph nodes by hipGraphNodeType: {kinds}")
    assert types and set(types) == {0}, kinds   # hipGraphNodeTypeKernel only
    # and the replay (instantiated on first use) gives the eager step's tokens
    for _ in range(2):
        got = g.run([20, 40], [[1, 2], [3, 4, 5]], [7, 8])
        want = _eager_tokens(model, [20, 40], [[1, 2], [3, 4, 5]], [7, 8], 4, 32)
        assert got == want
