"""hkv_decode_attn_noalloc (the decode entry point that allocates nothing; its scratch is a
static device array) against hkv_decode_attn with a caller workspace: bitwise equal
outputs under the fixed block schedule, on two calls in a row, the second smaller; across
launches whose (sequence, kv head) pair count changes (32, 8, 32 pairs), eagerly and with a
graph captured at one pair count and replayed after eager launches at another; and a
capacity error for a geometry beyond the scratch size."""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(seed, B, Hq, Hkv, sink, mid, rec):
    from heterokv import ops
    g = torch.Generator().manual_seed(seed)
    S = sink + mid + rec
    K = torch.randn((B, Hkv, S, 128), generator=g)
    K[..., [7, 31, 64, 100]] *= 8
    K = K.half()
    V = torch.randn((B, Hkv, S, 128), generator=g).half()
    q = (torch.randn((B, Hq, 128), generator=g) / math.sqrt(128)).half()
    zs = ops.F16Zone(B, Hkv, max(sink, 16), DEV)
    zs.write(K[:, :, :sink].to(DEV), V[:, :, :sink].to(DEV), 0)
    zr = ops.F16Zone(B, Hkv, rec, DEV)
    zr.write(K[:, :, sink + mid:].to(DEV), V[:, :, sink + mid:].to(DEV), 0)
    nb = (mid + 15) // 16
    perm = torch.randperm(B * nb, generator=g).to(torch.int32).reshape(B, nb)
    pool = ops.Int4Pool(B * nb, Hkv, DEV)
    ops.pack_tokens(pool, K[:, :, sink:sink + mid].to(DEV), V[:, :, sink:sink + mid].to(DEV), [0] * B, perm)
    pool.check_errors()
    return dict(q=q.to(DEV), zones=[(zs, None, sink), (zr, None, rec)], pool=pool, block_table=perm.to(DEV),
                int4_max_len=mid)


@pytest.mark.parametrize("handoff", [False, True])
def test_noalloc_matches_workspace_entry(handoff):
    from heterokv import ops
    cases = [("B=1 32/8, 64 + 28608 + 4096", _inputs(1, 1, 32, 8, 64, 28608, 4096)),
             ("B=2 28/4, 64 + 1500 + 700", _inputs(2, 2, 28, 4, 64, 1500, 700))]
    err = ops.ErrorWord(DEV)
    for name, c in cases:
        print("case: noalloc vs workspace, %s, agent_handoff=%s" % (name, handoff), flush=True)
        want = ops.decode_attention(workspace=ops.DecodeWorkspace(DEV, agent_handoff=handoff), deterministic=True,
                                    **c)
        got = ops.decode_attention(noalloc=True, agent_handoff=handoff, deterministic=True, err=err, **c)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        got2 = ops.decode_attention(noalloc=True, agent_handoff=handoff, deterministic=True, err=err, **c)
        torch.cuda.synchronize()
        assert torch.equal(got2, want)
    err.check()


def _fresh(c):
    from heterokv import ops
    return ops.decode_attention(workspace=ops.DecodeWorkspace(DEV), deterministic=True, **c)


@pytest.mark.parametrize("entry", ["noalloc", "shared_workspace"])
def test_pair_count_changes(entry):
    """One scratch (or one shared workspace) used by launches of 32, 8 and again 32 pairs:
    every output equals a fresh workspace's, bit for bit."""
    from heterokv import ops
    big = _inputs(4, 4, 32, 8, 64, 3000, 512)     # 4 x 8 = 32 pairs
    small = _inputs(5, 1, 32, 8, 64, 9000, 1024)  # 8 pairs, more ranges each
    ws = ops.DecodeWorkspace(DEV)
    err = ops.ErrorWord(DEV)
    want = {"big": _fresh(big), "small": _fresh(small)}
    for step, (name, c) in enumerate([("big", big), ("small", small), ("big", big), ("small", small)]):
        print("case: %s, launch %d, %s geometry" % (entry, step, name), flush=True)
        if entry == "noalloc":
            got = ops.decode_attention(noalloc=True, deterministic=True, err=err, **c)
        else:
            got = ops.decode_attention(workspace=ws, deterministic=True, err=err, **c)
        torch.cuda.synchronize()
        assert torch.equal(got, want[name])
    err.check()


def test_noalloc_graph_replay_across_pair_counts():
    """A graph that captured the allocation-free decode at 32 pairs, replayed after eager
    launches at 8 pairs (whose partial states land where nothing of the 32-pair launch's
    tickets lives), gives the eager 32-pair output on every replay."""
    from heterokv import ops
    big = _inputs(6, 4, 32, 8, 64, 3000, 512)
    small = _inputs(7, 1, 32, 8, 64, 9000, 1024)
    err = ops.ErrorWord(DEV)
    want_big, want_small = _fresh(big), _fresh(small)
    out = torch.empty_like(want_big)
    ops.decode_attention(noalloc=True, deterministic=True, err=err, out=out, **big)   # eager, 32 pairs
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        ops.decode_attention(noalloc=True, deterministic=True, err=err, out=out, **big)
    for rep in range(4):
        print("case: graph replay %d after an eager 8-pair launch" % rep, flush=True)
        got_small = ops.decode_attention(noalloc=True, deterministic=True, err=err, **small)
        torch.cuda.synchronize()
        assert torch.equal(got_small, want_small)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want_big)
    err.check()


def test_noalloc_rejects_oversized_geometry():
    from heterokv import HeteroKVError, ops
    c = _inputs(3, 2, 128, 8, 16, 64, 16)      # 16 pairs x 64 ranges x 16 heads: beyond 8 MB
    print("case: noalloc capacity error", flush=True)
    with pytest.raises(HeteroKVError, match="workspace"):
        ops.decode_attention(noalloc=True, splits=64, **c)
    with pytest.raises(HeteroKVError, match="takes no workspace"):
        from heterokv import _lib
        import ctypes
        a = _lib.DecodeArgs()
        a.workspace, a.workspace_bytes = 4096, 4096
        _lib.check(_lib.load().hkv_decode_attn_noalloc(ctypes.byref(a), None), "hkv_decode_attn_noalloc")
