"""The C-ABI library loads and exports every symbol include/heterokv.h declares;
argument errors come back as return codes with a message.  No GPU needed."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "heterokv.h")


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(hkv_[a-z0-9_]+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    from heterokv import _lib
    return _lib.load()


def test_header_symbols_exported(lib):
    names = _declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    from heterokv import _lib
    assert sorted(n for n, _, _ in _lib.SYMBOLS) == names


def test_version_and_record_size(lib):
    assert lib.hkv_abi_version() == 9
    assert lib.hkv_block_bytes(8, 128) == 17664
    assert lib.hkv_block_bytes(4, 128) == 8832
    assert lib.hkv_block_bytes(8, 64) == -1


def test_struct_layouts_match_c_compiler(tmp_path):
    """Every ctypes mirror has the size and field offsets gcc gives the C structs."""
    import shutil
    import subprocess
    from heterokv import _lib
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    structs = {"HkvPackArgs": _lib.PackArgs, "HkvRepackArgs": _lib.RepackArgs,
               "HkvZoneWriteArgs": _lib.ZoneWriteArgs, "HkvF16Zone": _lib.F16Zone,
               "HkvDecodeArgs": _lib.DecodeArgs, "HkvPrefillArgs": _lib.PrefillArgs,
               "HkvCopyDesc": _lib.CopyDesc, "HkvPfStats": _lib.PfStats, "HkvZoneStepArgs": _lib.ZoneStepArgs}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "%s"' % HEADER, "int main(void){"]
    for cname, py in structs.items():
        lines.append('printf("%s size %%zu\\n", sizeof(%s));' % (cname, cname))
        for fname, _ in py._fields_:
            lines.append('printf("%s %s %%zu\\n", offsetof(%s, %s));' % (cname, fname, cname, fname))
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, stdout=subprocess.PIPE, text=True).stdout.split("\n")
    got = {}
    for ln in out:
        if ln.strip():
            a, b, c = ln.split()
            got[(a, b)] = int(c)
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for fname, _ in py._fields_:
            assert got[(cname, fname)] == getattr(py, fname).offset, (cname, fname)


def test_argument_errors_are_reported(lib):
    rc = lib.hkv_quantize_groups(None, 0, 10, 0, None, None, None, None)
    assert rc == -1
    assert b"group_size" in lib.hkv_last_error()
    rc = lib.hkv_quantize_groups(None, 7, 10, 128, None, None, None, None)
    assert rc == -1 and b"dtype" in lib.hkv_last_error()
    assert lib.hkv_quantize_groups(None, 0, 0, 128, None, None, None, None) == 0
    assert lib.hkv_last_error() == b""


def test_decode_argument_errors(lib):
    from heterokv import _lib
    a = _lib.DecodeArgs()
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim = 1, 32, 8, 64
    assert lib.hkv_decode_attn(ctypes.byref(a), None) == -4
    a.head_dim = 128
    a.num_q_heads = 30
    assert lib.hkv_decode_attn(ctypes.byref(a), None) == -1
    a.num_q_heads = 32 * 8 * 4
    assert lib.hkv_decode_attn(ctypes.byref(a), None) == -4  # n_rep > 16
    # workspace too small -> capacity error, before any launch
    a.num_q_heads = 32
    a.q = a.out = a.workspace = 4096
    a.workspace_bytes = 16
    a.num_f16_zones = 1
    a.f16[0] = _lib.F16Zone(k=4096, v=4096, capacity=64, max_len=64, lens=None)
    assert lib.hkv_decode_attn(ctypes.byref(a), None) == -3
    assert b"workspace" in lib.hkv_last_error()
    a.f16[0] = _lib.F16Zone(k=4096, v=4096, capacity=64, max_len=80, lens=None)
    assert lib.hkv_decode_attn(ctypes.byref(a), None) == -1
    # range bounds are 32-bit: at most 2^26 INT4 tokens per sequence
    a.f16[0] = _lib.F16Zone(k=4096, v=4096, capacity=64, max_len=64, lens=None)
    a.int4_max_len = (1 << 26) + 1
    assert lib.hkv_decode_attn(ctypes.byref(a), None) == -1
    assert b"int4_max_len" in lib.hkv_last_error()


def test_workspace_size(lib):
    from heterokv import ops
    n = ops.decode_workspace_bytes(1, 32, 8, 28608, [64, 4096])
    # header + a fixed ticket area for 1024 pairs (one 256-byte agent line with the ticket
    # and the XCD mask, one 256-byte XCD-local line each) + partial states for up to 64
    # ranges per (sequence, kv head): 8 pairs x 64 ranges x 4 heads x 132 floats
    assert n == 256 + 1024 * 256 + 1024 * 256 + 8 * 64 * 4 * 132 * 4
    # the ticket area does not move with the geometry
    n2 = ops.decode_workspace_bytes(4, 32, 8, 28608, [64, 4096])
    assert n2 - n == 24 * 64 * 4 * 132 * 4


def test_prefetcher_and_gather_argument_errors(lib):
    from heterokv import _lib
    assert lib.hkv_pf_submit(None, None, 0, 0, 0) == -1
    assert b"null" in lib.hkv_last_error()
    assert lib.hkv_pf_wait(None, 0, None) == -1
    assert lib.hkv_pf_mark(None, 0, None) == -1
    assert lib.hkv_pf_record(None, 0) == -1
    st = _lib.PfStats()
    assert lib.hkv_pf_stats(None, ctypes.byref(st)) == -1
    assert lib.hkv_pf_host_ptr(None, 0) is None
    assert lib.hkv_pf_stream(None) is None
    assert lib.hkv_pf_destroy(None) == 0
    out = ctypes.c_void_p()
    assert lib.hkv_pf_create(0, 0, 0, ctypes.byref(out)) == -1     # num_slots must be >= 1
    # gather: empty is a no-op, bad record size / null buffers are argument errors
    assert lib.hkv_gather_blocks(None, 0, None, 0, None, 0, 8832, None, None, None) == 0
    assert lib.hkv_gather_blocks(4096, 4, None, 0, 4096, 2, 8830, 4096, None, None) == -1
    assert lib.hkv_gather_blocks(4096, 4, None, 2, 4096, 2, 8832, 4096, None, None) == -1


def _err(lib, rc, code, text):
    assert rc == code, (rc, lib.hkv_last_error())
    assert text in lib.hkv_last_error(), lib.hkv_last_error()


def test_pack_and_unpack_argument_errors(lib):
    from heterokv import _lib
    a = _lib.PackArgs()
    a.batch, a.num_kv_heads, a.head_dim, a.num_tokens, a.dtype = 1, 8, 64, 16, 0
    _err(lib, lib.hkv_pack_tokens(ctypes.byref(a), None), -4, b"head_dim")
    a.head_dim = 128
    a.dtype = 2                                     # fp32 K/V are not packed (the reference's K/V are fp16/bf16)
    _err(lib, lib.hkv_pack_tokens(ctypes.byref(a), None), -1, b"dtype")
    a.dtype = 0
    a.num_kv_heads = 0
    _err(lib, lib.hkv_pack_tokens(ctypes.byref(a), None), -1, b"hkv_pack_tokens")
    a.num_kv_heads = 8
    _err(lib, lib.hkv_pack_tokens(ctypes.byref(a), None), -1, b"hkv_pack_tokens")   # null pointers
    a.k = a.v = a.start_pos = a.block_table = a.pool = 4096
    a.bt_stride, a.pool_blocks = 1, 0
    _err(lib, lib.hkv_pack_tokens(ctypes.byref(a), None), -1, b"empty")
    # unpack(pool, pool_blocks, block_table, num_kv_heads, head_dim, num_tokens, which, codes, scales, zps, stream)
    _err(lib, lib.hkv_unpack_tokens(4096, 1, 4096, 8, 64, 16, 0, None, None, None, None), -4, b"head_dim")
    _err(lib, lib.hkv_unpack_tokens(4096, 1, 4096, 8, 128, 16, 2, None, None, None, None), -1, b"which")
    _err(lib, lib.hkv_unpack_tokens(4096, 1, 4096, 0, 128, 16, 0, None, None, None, None), -1, b"sizes")
    _err(lib, lib.hkv_unpack_tokens(None, 1, 4096, 8, 128, 16, 0, None, None, None, None), -1, b"null")
    _err(lib, lib.hkv_unpack_tokens(4096, 1, 4096, 8, 128, 16, 0, 4097, None, None, None), -1, b"hkv_unpack_tokens")
    # dequantize_groups(codes, scales, zps, n, group_size, out, out_dtype, stream)
    _err(lib, lib.hkv_dequantize_groups(4096, 4096, 4096, 128, 0, 4096, 0, None), -1, b"group_size")
    _err(lib, lib.hkv_dequantize_groups(4096, 4096, 4096, 128, 128, 4096, 9, None), -1, b"hkv_dequantize_groups")
    _err(lib, lib.hkv_dequantize_groups(None, 4096, 4096, 128, 128, 4096, 0, None), -1, b"null")


def test_prefill_argument_errors(lib):
    from heterokv import _lib
    a = _lib.PrefillArgs()
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.num_queries = 1, 32, 8, 64, 4
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -4, b"head_dim")
    a.head_dim = 128
    a.num_q_heads = 30
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -1, b"multiple")
    a.num_q_heads = 32
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -1, b"null q/out")
    a.q, a.out = 4098, 8192                        # q not 16-byte aligned
    a.q_stride_b, a.q_stride_h, a.q_stride_t = 32 * 4 * 128, 4 * 128, 128
    a.out_stride_b, a.out_stride_h, a.out_stride_t = 32 * 4 * 128, 4 * 128, 128
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -1, b"16-byte")
    a.q = 4096
    a.chunk_k = 16384                              # chunk K without chunk V
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -1, b"both")
    a.chunk_k = None
    a.int4_max_len = -1
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -1, b"int4_max_len")
    a.int4_max_len = 100
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -1, b"block table")
    a.block_table, a.pool, a.pool_blocks, a.bt_stride = 4096, 65536, 8, 6   # 6 blocks hold 96 < 100 tokens
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -3, b"stride")
    a.bt_stride = 7
    a.num_f16_zones = 1
    a.f16[0] = _lib.F16Zone(k=4096, v=4096, capacity=64, max_len=65, lens=None)
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -1, b"zone 0")
    a.f16[0] = _lib.F16Zone(k=4100, v=4096, capacity=64, max_len=64, lens=None)
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -1, b"misaligned")
    # INT4 and zone keys: the zone kernel's state needs a workspace of the documented size
    # (state rows, then the chunk's K rows and V tiles at 16-token capacity)
    a.f16[0] = _lib.F16Zone(k=4096, v=4096, capacity=64, max_len=64, lens=None)
    need = lib.hkv_prefill_workspace_bytes(1, 32, 4)
    assert need == 1 * 32 * 4 * 132 * 4 + 2 * 32 * 16 * 128 * 2 and lib.hkv_prefill_workspace_bytes(0, 32, 4) == 0
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -1, b"workspace")
    a.workspace, a.workspace_bytes = 1 << 20, need - 1
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -1, b"workspace")
    # a causal chunk alone needs it too (its K/V are rewritten in the zone layout)
    a.num_f16_zones, a.int4_max_len, a.workspace, a.workspace_bytes = 0, 0, None, 0
    a.chunk_k, a.chunk_v = 16384, 16384
    _err(lib, lib.hkv_prefill_attn(ctypes.byref(a), None), -1, b"workspace")


def test_zone_and_scoring_argument_errors(lib):
    from heterokv import _lib
    w = _lib.ZoneWriteArgs()
    w.batch, w.num_kv_heads, w.head_dim, w.num_tokens, w.capacity = 1, 8, 64, 4, 64
    _err(lib, lib.hkv_zone_write(ctypes.byref(w), None), -4, b"head_dim")
    w.head_dim, w.capacity = 128, 60                 # capacity must be a multiple of 16
    _err(lib, lib.hkv_zone_write(ctypes.byref(w), None), -1, b"hkv_zone_write")
    w.capacity = 64
    _err(lib, lib.hkv_zone_write(ctypes.byref(w), None), -1, b"hkv_zone_write")   # null pointers
    w.k = w.v = w.zone_k = w.zone_v = 4096
    w.ring = 65                                      # ring longer than the zone
    _err(lib, lib.hkv_zone_write(ctypes.byref(w), None), -1, b"hkv_zone_write")
    # zone_read(zone_k, zone_v, batch, num_kv_heads, head_dim, capacity, n, out_k, out_v, stream)
    _err(lib, lib.hkv_zone_read(4096, 4096, 1, 8, 64, 64, 4, 4096, 4096, None), -4, b"head_dim")
    _err(lib, lib.hkv_zone_read(4096, 4096, 1, 8, 128, 64, 65, 4096, 4096, None), -1, b"hkv_zone_read")
    _err(lib, lib.hkv_zone_read(4096, 4096, 1, 8, 128, 64, 4, None, None, None), -1, b"null")
    # zone_copy(src_k, src_v, src_cap, src_slot, dst_k, dst_v, dst_cap, dst_slot, batch, heads, head_dim, n, stream)
    _err(lib, lib.hkv_zone_copy(4096, 4096, 64, 0, 8192, 8192, 64, 0, 1, 8, 64, 4, None), -4, b"head_dim")
    _err(lib, lib.hkv_zone_copy(4096, 4096, 64, 62, 8192, 8192, 64, 0, 1, 8, 128, 4, None), -3, b"slot range")
    _err(lib, lib.hkv_zone_copy(None, 4096, 64, 0, 8192, 8192, 64, 0, 1, 8, 128, 4, None), -1, b"null")
    # attn_weights(scores, sb, sh, stats, batch, heads, n_items, order, out, out_stride_b, accumulate, stream)
    _err(lib, lib.hkv_attn_weights(4096, 64, 64, 4096, 0, 4, 64, None, 4096, 64, 0, None), -1, b"sizes")
    _err(lib, lib.hkv_attn_weights(None, 64, 64, 4096, 1, 4, 64, None, 4096, 64, 0, None), -1, b"null")
    _err(lib, lib.hkv_attn_weights(4096, 64, 64, 4096, 1, 4, 64, None, 4096, 32, 0, None), -1, b"stride")
    # block_scores(token_scores, seq_len, block_size, out, stream)
    _err(lib, lib.hkv_block_scores(4096, 64, 0, 4096, None), -1, b"sizes")
    _err(lib, lib.hkv_block_scores(None, 64, 16, 4096, None), -1, b"null")
    # eviction_candidates(scores, seq_len, block_size, sink, window, max_blocks, out, num_out, ws, ws_bytes, stream)
    n = ctypes.c_int32()
    _err(lib, lib.hkv_eviction_candidates(4096, 64, 0, 0, 0, 4, 4096, ctypes.byref(n), 4096, 1 << 20, None), -1,
         b"hkv_eviction_candidates")
    _err(lib, lib.hkv_eviction_candidates(4096, 64, 16, 0, 0, 4, 4096, None, 4096, 1 << 20, None), -1, b"num_out")
    need = lib.hkv_eviction_workspace_bytes(4096, 16, 0, 0, 4)
    assert need > 0
    _err(lib, lib.hkv_eviction_candidates(4096, 4096, 16, 0, 0, 4, 4096, ctypes.byref(n), 4096, need - 8, None), -3,
         b"workspace")


def test_repack_and_zone_step_argument_errors(lib):
    from heterokv import _lib
    r = _lib.RepackArgs()
    r.batch, r.num_kv_heads, r.head_dim, r.num_tokens, r.zp_dtype = 1, 8, 64, 16, 3
    _err(lib, lib.hkv_repack_codes(ctypes.byref(r), None), -4, b"head_dim")
    r.head_dim, r.zp_dtype = 128, 0                 # zero points are uint8 or float32
    _err(lib, lib.hkv_repack_codes(ctypes.byref(r), None), -1, b"zp dtype")
    r.zp_dtype = 3
    _err(lib, lib.hkv_repack_codes(ctypes.byref(r), None), -1, b"null")
    r.num_tokens = 0
    assert lib.hkv_repack_codes(ctypes.byref(r), None) == 0   # nothing to do
    z = _lib.ZoneStepArgs()
    z.batch, z.num_kv_heads, z.head_dim = 1, 8, 64
    _err(lib, lib.hkv_zone_step(ctypes.byref(z), None), -4, b"head_dim")
    z.head_dim = 128
    _err(lib, lib.hkv_zone_step(ctypes.byref(z), None), -1, b"null")
    z.k = z.v = z.tail_k = z.tail_v = z.state = 4096
    z.tail_capacity, z.tail_ring = 64, 80           # ring longer than the tail zone
    _err(lib, lib.hkv_zone_step(ctypes.byref(z), None), -1, b"tail ring")
    z.tail_ring = 64
    z.hh_budget, z.hh_capacity = 32, 16             # heavy-hitter zone smaller than its budget
    _err(lib, lib.hkv_zone_step(ctypes.byref(z), None), -1, b"heavy-hitter")
