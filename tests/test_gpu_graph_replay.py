"""Graph capture of the decode ops: the absorbed-MLA decode, the DSA
selection with its sparse contraction, and the position-free attention are
captured once in a HIP graph and replayed three times, with eager calls of
the same ops on other inputs and synchronizations between the replays; every
replay must equal the eager result bit for bit (no memset nodes, workspaces
and tables that keep their addresses)."""
import pytest
import torch

from voom_amd import ops, synthetic

pytestmark = pytest.mark.gpu


def bits(t):
    return t.contiguous().view(torch.int16) if t.dtype == torch.bfloat16 else t


def replay_matches_eager(run, disturb):
    eager = [t.clone() for t in run()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            outs = run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    # the graph holds the workspaces' addresses: keep every one alive even if
    # an eager call below were to replace it with a larger one
    keep = list(ops._WORKSPACES.values())
    for rep in range(3):
        for t in outs:
            t.zero_()
        disturb()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(bits(a), bits(b)), f"replay {rep} differs from the eager result"
    del keep


def test_mla_decode_replays():
    print("[graph] absorbed MLA decode", flush=True)
    a = synthetic.mla_decode_inputs(batch=2, ctx=3000, seed=31)
    b = synthetic.mla_decode_inputs(batch=2, ctx=1500, seed=32)
    w_uk, w_uv_t = ops.split_kv_b(a.kv_b, 128, a.dn, a.dv)
    w_uk, w_uv_t = ops.pack_head_weights(w_uk), ops.pack_head_weights(w_uv_t)

    def run(x=a):
        return [ops.mla_absorbed_decode(x.q_nope, x.q_rope, x.lat_pool, x.block_table,
                                        x.ctx_lens, w_uk, w_uv_t, scale=x.scale)]

    replay_matches_eager(run, lambda: run(b))


def test_dsa_selection_and_sparse_contraction_replay():
    print("[graph] DSA scores + top-k + sparse MLA", flush=True)
    g = torch.Generator(device="cuda").manual_seed(33)
    S, K = 20000, 512
    keys = [(torch.randn((1, S, 128), generator=g, device="cuda") * 0.5).to(torch.bfloat16)
            for _ in range(2)]
    q_idx = (torch.randn((1, 32, 128), generator=g, device="cuda")).to(torch.bfloat16)
    w_head = torch.rand((1, 32), generator=g, device="cuda")
    lens = torch.tensor([S], dtype=torch.int32, device="cuda")
    scores = torch.empty((1, S), dtype=torch.float32, device="cuda")
    sel = torch.empty((1, K), dtype=torch.int32, device="cuda")
    sel_lens = torch.empty((1,), dtype=torch.int32, device="cuda")
    lat = synthetic.mla_decode_inputs(batch=1, ctx=S, seed=34)
    q_lat = torch.cat([(torch.randn((1, 128, 512), generator=g, device="cuda") * 0.05),
                       lat.q_rope.float()], -1).to(torch.bfloat16)

    def run(i=0):
        ops.dsa_index_scores(q_idx, w_head, keys[i], lens, scale=128 ** -0.5, out=scores)
        ops.dsa_topk(scores, lens, K, sel=sel, sel_lens=sel_lens)
        out = ops.mla_sparse_decode(q_lat, lat.lat_pool, lat.block_table, sel, sel_lens,
                                    scale=lat.scale)
        return [sel, sel_lens, out]

    replay_matches_eager(run, lambda: run(1))


def test_position_free_attention_replays():
    print("[graph] position-free attention", flush=True)
    g = torch.Generator(device="cuda").manual_seed(35)
    P, NKV, NQ, D, TK = 3000, 8, 32, 128, 2500
    kp = [(torch.randn((P, NKV, 1, D), generator=g, device="cuda")).to(torch.bfloat16)
          for _ in range(2)]
    vp = [(torch.randn((P, NKV, 1, D), generator=g, device="cuda")).to(torch.bfloat16)
          for _ in range(2)]
    table = torch.randint(0, P, (TK,), generator=g, device="cuda", dtype=torch.int32)
    kpos = torch.arange(TK, dtype=torch.int32, device="cuda")
    qpos = torch.tensor([TK - 1], dtype=torch.int32, device="cuda")
    q = torch.randn((1, NQ, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    cos, sin = ops.rope_cache(TK, D, 10000.0, device="cuda")

    def run(i=0):
        return [ops.position_free_paged_attention(q, kp[i], vp[i], table, kpos, qpos, cos, sin,
                                                  scale=D ** -0.5)]

    replay_matches_eager(run, lambda: run(1))


def test_launch_stream_follows_torch_current_stream():
    """Every op launches on the stream ops._stream(None) names: torch's current
    stream, inside a stream context and under graph capture too (there the
    capturing stream, or the launches would escape the graph)."""
    print("[graph] launch stream lookup", flush=True)
    assert ops._stream(None) == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert ops._stream(None) == side.cuda_stream
    seen = []
    x = torch.zeros(16, device="cuda")
    torch.cuda.synchronize()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            seen.append((ops._stream(None), torch.cuda.current_stream().cuda_stream))
            x.add_(1)
    torch.cuda.current_stream().wait_stream(cap)
    assert seen[0][0] == seen[0][1] == cap.cuda_stream
    graph.replay()
    torch.cuda.synchronize()
    assert float(x[0]) == 1.0
