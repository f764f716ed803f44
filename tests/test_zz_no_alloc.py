"""voom_paged_gqa_decode_noalloc against voom_paged_gqa_decode, through the C ABI.

The no-alloc entry point runs the same kernels with the split partials in a
file-scope device array instead of a caller workspace, so its output must be
bit-identical to the workspace entry point's for the same inputs and split
count.  Two calls in a row, the second smaller, check that nothing left in the
array by the first call leaks into the second.
"""
import numpy as np
import pytest
import torch

from oracle import paged_attention as opa
from voom_amd import _lib, ops, synthetic

pytestmark = pytest.mark.gpu


def entry():
    return _lib.lib().voom_paged_gqa_decode_noalloc


def max_bytes():
    return _lib.lib().voom_paged_gqa_noalloc_max_bytes()


def noalloc(inp, out, lse, num_splits):
    B, NQ, D = inp.q.shape
    slots, NKV, PT, _ = inp.k_pool.shape
    max_pages = inp.block_table.shape[1]
    return entry()(
        inp.q.data_ptr(), inp.k_pool.data_ptr(), inp.v_pool.data_ptr(),
        inp.block_table.data_ptr(), inp.ctx_lens.data_ptr(), out.data_ptr(), lse.data_ptr(),
        B, NQ, NKV, D, PT, max_pages, slots, inp.scale, num_splits,
        torch.cuda.current_stream().cuda_stream)


def with_workspace(inp, num_splits):
    B, NQ, D = inp.q.shape
    slots, NKV, PT, _ = inp.k_pool.shape
    need = ops.gqa_workspace_bytes(B, NQ, NKV, D, num_splits)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    out = torch.empty_like(inp.q)
    lse = torch.empty((B, NQ), dtype=torch.float32, device="cuda")
    _lib.call("voom_paged_gqa_decode", inp.q.data_ptr(), inp.k_pool.data_ptr(),
              inp.v_pool.data_ptr(), inp.block_table.data_ptr(), inp.ctx_lens.data_ptr(),
              out.data_ptr(), lse.data_ptr(), ws.data_ptr(), need, B, NQ, NKV, D, PT,
              inp.block_table.shape[1], slots, inp.scale, num_splits,
              torch.cuda.current_stream().cuda_stream)
    return out, lse


def test_noalloc_matches_the_workspace_entry_point_twice():
    cases = [
        # config-2 geometry, long contexts, the library's split count
        dict(batch=16, ctx_lens=None, num_q_heads=32, num_kv_heads=8, head_dim=128, splits=0,
             seed=31),
        # smaller second call: fewer sequences, explicit split count, D = 64
        dict(batch=3, ctx_lens=[1, 700, 5000], num_q_heads=8, num_kv_heads=2, head_dim=64,
             splits=64, seed=32),
    ]
    for c in cases:
        print(f"[noalloc] B={c['batch']} NQ={c['num_q_heads']} NKV={c['num_kv_heads']} "
              f"D={c['head_dim']} splits={c['splits']}", flush=True)
        kw = dict(batch=c["batch"], num_q_heads=c["num_q_heads"],
                  num_kv_heads=c["num_kv_heads"], head_dim=c["head_dim"], page_tokens=64,
                  seed_base=c["seed"], device="cuda")
        if c["ctx_lens"] is not None:
            kw["ctx_lens"] = c["ctx_lens"]
        inp = synthetic.gqa_decode_inputs(**kw)
        want, want_lse = with_workspace(inp, c["splits"])
        out = torch.empty_like(inp.q)
        lse = torch.empty_like(want_lse)
        assert noalloc(inp, out, lse, c["splits"]) == 0, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
        assert torch.equal(lse, want_lse)
        pick = [0, inp.q.shape[0] - 1]
        q, k, v = synthetic.to_reference_layout(inp)
        ref = opa.paged_decode(q[pick], k, v, inp.table_host[pick], inp.ctx_host[pick],
                               inp.scale)
        np.testing.assert_allclose(out[pick].float().cpu().numpy(), ref, atol=2e-2, rtol=1e-2)


def test_noalloc_rejects_partials_beyond_its_array():
    print("[noalloc] oversize request", flush=True)
    inp = synthetic.gqa_decode_inputs(batch=2, ctx_lens=[10, 20], num_q_heads=8,
                                      num_kv_heads=2, head_dim=128, page_tokens=64,
                                      seed_base=33, device="cuda")
    out = torch.empty_like(inp.q)
    lse = torch.empty((2, 8), dtype=torch.float32, device="cuda")
    limit = max_bytes()
    assert limit == 16 << 20
    rc = noalloc(inp, out, lse, 1 << 20)  # 1M splits need far more than the array
    assert rc == _lib.VOOM_EINVAL
    assert "scratch" in _lib.last_error()


def _graph_case(seed):
    return synthetic.gqa_decode_inputs(batch=4, ctx_lens=[33, 900, 2049, 64], num_q_heads=16,
                                       num_kv_heads=4, head_dim=128, page_tokens=64,
                                       seed_base=seed, device="cuda")


def test_noalloc_replays_from_a_captured_graph():
    """The entry point's reason to exist: a call captured in a HIP graph and
    replayed.  Three replays, each after eager workspace calls on other
    inputs; every replay is bit-equal to the eager workspace result."""
    print("[noalloc] graph capture + replays", flush=True)
    inp = _graph_case(41)
    other = _graph_case(42)
    want, want_lse = with_workspace(inp, 0)
    out = torch.empty_like(inp.q)
    lse = torch.empty_like(want_lse)
    assert noalloc(inp, out, lse, 0) == 0, _lib.last_error()  # warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out.zero_()
        with torch.cuda.graph(g, stream=s):
            assert noalloc(inp, out, lse, 0) == 0, _lib.last_error()
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        out.zero_()
        lse.zero_()
        with_workspace(other, 0)
        assert noalloc(other, torch.empty_like(out), torch.empty_like(lse), 64) == 0
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
        assert torch.equal(lse, want_lse)


_FIRST_CALL_IN_CAPTURE = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from tests.test_zz_no_alloc import _graph_case, noalloc, with_workspace
from voom_amd import _lib
inp = _graph_case(43)
out = torch.empty_like(inp.q)
lse = torch.empty((inp.q.shape[0], inp.q.shape[1]), dtype=torch.float32, device="cuda")
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
s = torch.cuda.Stream()
with torch.cuda.stream(s):
    with torch.cuda.graph(g, stream=s):
        rc = noalloc(inp, out, lse, 0)   # the process's first call of the entry point
assert rc == 0, _lib.last_error()
torch.cuda.synchronize()
want, want_lse = with_workspace(inp, 0)
for _ in range(2):
    out.zero_()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    assert torch.equal(lse, want_lse)
print("FIRST_CALL_IN_CAPTURE_OK", flush=True)
"""


def test_noalloc_first_call_inside_a_capture():
    """A fresh process whose first call of the entry point is made under graph
    capture (the scratch array's address is resolved inside the capture)."""
    import subprocess
    import sys
    from pathlib import Path

    print("[noalloc] first call under capture, fresh process", flush=True)
    root = str(Path(__file__).resolve().parent.parent)
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE, root], cwd=root,
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and "FIRST_CALL_IN_CAPTURE_OK" in res.stdout, (
        res.stdout[-2000:] + res.stderr[-3000:])
