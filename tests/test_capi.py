"""CPU tests of the boundary: the C-ABI library loads, exports every symbol include/q3attn.h
declares, rejects bad arguments with error codes and messages (no kernel is launched), and the
Python entry points refuse CPU tensors instead of falling back to anything."""
import ctypes
import os
import re

import pytest
import torch

import q3attn
from q3attn import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q3attn.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(q3a_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = _declared()
    assert "q3a_paged_decode" in names and "q3a_cp_attn" in names
    for n in names:
        assert hasattr(L, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert L.q3a_abi_version() == _lib.ABI_VERSION


def _decode(**kw):
    args = dict(q=16, q_sb=2048, q_sh=128, k=16, v=16, sp=16384, st=1024, sh=128, num_pages=8, page=16,
                seqlens=16, bt=16, bt_sb=4, max_pages=4, out=16, o_sb=2048, o_sh=128, ws=16, ws_bytes=1 << 30,
                B=2, Hq=16, Hkv=8, D=128, scale=0.088, split=0)
    args.update(kw)
    L = _lib.lib()
    return L.q3a_paged_decode(args["q"], args["q_sb"], args["q_sh"], args["k"], args["v"], args["sp"], args["st"],
                              args["sh"], args["num_pages"], args["page"], args["seqlens"], args["bt"],
                              args["bt_sb"], args["max_pages"], args["out"], args["o_sb"], args["o_sh"],
                              args["ws"], args["ws_bytes"], args["B"], args["Hq"], args["Hkv"], args["D"],
                              args["scale"], args["split"], None)


@pytest.mark.parametrize("kw,frag", [
    (dict(D=64), "head_dim"),
    (dict(Hq=8), "num_q_heads"),
    (dict(Hkv=32, Hq=64), "num_kv_heads"),
    (dict(page=24), "page_size"),
    (dict(q=None), "null pointer"),
    (dict(q=18), "aligned"),
    (dict(st=1020), "strides"),
    (dict(split=40), "split_tokens"),
    (dict(max_pages=4096, split=16), "splits exceed"),
    (dict(split=2048), "exceeds 1024"),
    (dict(sh=-128), "page extent"),
    (dict(q_sh=1 << 30), "q head stride"),
    (dict(q_sh=-128), "q head stride"),
    (dict(ws_bytes=10, max_pages=16, B=65), "workspace"),  # 65 rows of a 256-token table: stream-K, with workspace
    (dict(ws_bytes=10, max_pages=16, B=4), "workspace"),   # 4 rows of a 256-token table: chunks, with workspace
    (dict(B=-1), "batch"),
    (dict(split=-5), "split_tokens"),                      # not a path code
    (dict(split=-4, B=65, max_pages=16), "not a decode plan"),  # planned, with a workspace no plan was built in
    (dict(split=-1, max_pages=129), "decode path"),        # the row kernel takes tables of at most 2,048 tokens
    (dict(split=-3, B=4097), "decode path"),               # stream-K takes at most 4,096 rows
    (dict(split=-2, max_pages=8193), "decode path"),       # chunks: at most 64 tiles per wave
])
def test_paged_decode_rejects_bad_arguments(kw, frag):
    rc = _decode(**kw)
    assert rc < 0
    assert frag in _lib.lib().q3a_last_error().decode()


def test_paged_decode_empty_batch_is_a_noop():
    assert _decode(B=0) == 0


def test_workspace_and_default_split():
    L = _lib.lib()
    # 576-row shape: 576 rows, 113 pages of 16 tokens
    split = L.q3a_paged_decode_default_split(576, 8, 113, 16)
    assert split % 16 == 0 and split >= 16
    n_splits = -(-113 * 16 // split)
    assert n_splits <= 64
    # one 528-byte partial record (2 x 128 16-bit o values, m[2], l[2] in fp32) per (row, split, KV head)
    assert L.q3a_paged_decode_workspace_bytes(576, 16, 8, 128, 113, 16, split) == 576 * n_splits * 8 * 528
    # one split: no workspace
    assert L.q3a_paged_decode_workspace_bytes(4, 16, 8, 128, 4, 16, 64) == 0
    # the row-parallel path (tables up to 128 tokens, or up to 64 rows of up to 2,048 tokens): no workspace
    assert L.q3a_paged_decode_workspace_bytes(4096, 16, 8, 128, 8, 16, 0) == 0
    assert L.q3a_paged_decode_workspace_bytes(64, 16, 8, 128, 128, 16, 0) == 0
    assert L.q3a_paged_decode_workspace_bytes(65, 16, 8, 128, 128, 16, 0) > 0
    assert L.q3a_paged_decode_workspace_bytes(64, 16, 8, 128, 129, 16, 0) > 0
    # small batches get smaller splits (more workgroups)
    assert L.q3a_paged_decode_default_split(1, 8, 4, 16) == 16


def test_workspace_of_the_decode_paths():
    """Up to 16 rows of tables of 256 tokens or more take the chunked kernel: one 1,040-byte fp32 record (o[2][128],
    m[2], l[2]) per (row, chunk, KV head), 16 chunks of 128 tokens up to 2,048-token tables, of 256 tokens up to
    4,096, then 8 waves of several tiles; a table held by one chunk needs no records.  The path codes force a kernel."""
    L = _lib.lib()
    ws = lambda B, pages, split: L.q3a_paged_decode_workspace_bytes(B, 16, 8, 128, pages, 16, split)
    rec = 1040
    assert ws(4, 128, 0) == 4 * 16 * 8 * rec                      # auto: chunks, 16 x 128 tokens
    assert ws(4, 128, -2) == 4 * 16 * 8 * rec
    assert ws(4, 128, -1) == 0                                    # forced row kernel: one launch
    assert ws(4, 256, 0) == 4 * 16 * 8 * rec                      # 16 x 256 tokens
    assert ws(4, 512, 0) == 4 * 16 * 8 * rec                      # 16 x (8 waves x 4 tiles)
    assert ws(4, 300, -2) == 4 * 13 * 8 * rec                     # 8 waves x 3 tiles: ceil(300 / 24) chunks
    assert ws(16, 16, 0) == 16 * 2 * 8 * rec                      # 256-token tables: two chunks
    assert ws(1, 8, -2) == 0                                      # one chunk: no records
    assert ws(17, 16, 0) == 0                                     # 17 rows: the row-parallel kernel
    assert ws(4, 15, 0) == 0                                      # 240-token tables: the row-parallel kernel
    assert ws(4, 128, -3) > 0 and ws(4, 128, -3) != ws(4, 128, 0)  # forced stream-K
    assert ws(4, 129, -1) == 0                                    # a code that does not take the shape: nothing


def _plan(**kw):
    a = dict(seqlens=256, bt=256, bt_sb=16, bt_st=65 * 16, tables=1, max_pages=16, page=16, B=65, Hkv=8,
             form=0, plans=256, stride=1 << 24, plans_bytes=1 << 30)
    a.update(kw)
    return _lib.lib().q3a_paged_decode_plan(a["seqlens"], a["bt"], a["bt_sb"], a["bt_st"], a["tables"],
                                            a["max_pages"], a["page"], a["B"], a["Hkv"], a["form"], a["plans"],
                                            a["stride"], a["plans_bytes"], None)


@pytest.mark.parametrize("kw,frag", [
    (dict(form=3), "form"), (dict(form=-1), "form"), (dict(seqlens=None), "null"), (dict(plans=None), "null"),
    (dict(tables=0), "num_tables"), (dict(plans=264), "256-byte"), (dict(tables=2, stride=1000), "256-byte"),
    (dict(tables=2, stride=256), "256-byte"), (dict(plans_bytes=100), "bytes"),
    (dict(bt_sb=8), "overlap"), (dict(tables=2, bt_st=16), "overlap"),
    (dict(B=8), "no plan"),                  # 8 rows of a 256-token table: the chunked kernel, no plan
    (dict(B=65, max_pages=8), "no plan"),    # 128-token tables: the row-parallel kernel
    (dict(Hkv=4), "no plan"), (dict(B=4097), "no plan"), (dict(page=24), "no plan"), (dict(page=8192), "no plan"),
])
def test_decode_plan_rejects_bad_arguments(kw, frag):
    rc = _plan(**kw)
    assert rc < 0
    assert frag in _lib.lib().q3a_last_error().decode()


def test_decode_plan_bytes_follow_the_library_choice():
    """Plans exist exactly for the shapes the library decodes with stream-K; a plan is a stream-K workspace (prefix
    sums, slot pages, partial records of the grid the call launches) plus the ranges, the first tile lists and 8 B
    per tile of the table capacity."""
    L = _lib.lib()
    pb = lambda B, pages, page=16, hkv=8: L.q3a_paged_decode_plan_bytes(B, hkv, pages, page)
    assert pb(8, 16) == 0 and pb(16, 129) == 0        # chunks
    assert pb(64, 128) == 0 and pb(4096, 8) == 0       # row-parallel
    assert pb(4097, 16) == 0 and pb(576, 129, hkv=4) == 0
    for B, pages in ((65, 16), (17, 129), (576, 129), (4096, 64)):
        assert pb(B, pages) >= 4 * (2 * B + 1) + B * pages * 8, (B, pages)
        assert pb(B, pages) % 256 == 0
    assert pb(576, 258, page=8 * 16) == pb(576, 258 * 8)  # only the capacity in tokens matters


@pytest.mark.parametrize("kw,frag", [
    (dict(n_live=0), "n_live"), (dict(n_live=17), "n_live"), (dict(D=64), "head_dim"),
    (dict(Hq=12), "num_q_heads"), (dict(q=None), "null"), (dict(k_ss=100), "strides"), (dict(v_sh=4), "strides"),
    (dict(k_ss=64), "slot strides"), (dict(v_ss=64), "slot strides"), (dict(v_ss=(1 << 26) + 8), "slot strides"),
])
def test_cp_attn_rejects_bad_arguments(kw, frag):
    a = dict(q=16, q_sb=2048, k=16, k_sb=16384, k_sh=2048, k_ss=128, v=16, v_sb=32768, v_sh=4096, v_ss=256, out=16,
             o_sb=2048, B=4, Hq=16, Hkv=8, D=128, n_live=3, scale=0.088)
    a.update(kw)
    rc = _lib.lib().q3a_cp_attn(a["q"], a["q_sb"], a["k"], a["k_sb"], a["k_sh"], a["k_ss"], a["v"], a["v_sb"],
                                a["v_sh"], a["v_ss"], a["out"], a["o_sb"], a["B"], a["Hq"], a["Hkv"], a["D"],
                                a["n_live"], a["scale"], None)
    assert rc < 0 and frag in _lib.lib().q3a_last_error().decode()


@pytest.mark.parametrize("kw,frag", [
    (dict(kn=None), "k_new"), (dict(vn=None), "k_new"), (dict(kn=18), "aligned"), (dict(vn_sb=1030), "strides"),
    (dict(n_live=0), "n_live"), (dict(Hq=8), "num_q_heads"), (dict(v=24), "aligned"),
])
def test_cp_attn_append_rejects_bad_arguments(kw, frag):
    a = dict(q=16, q_sb=2048, kn=16, kn_sb=1024, vn=16, vn_sb=4096, k=16, k_sb=16384, k_sh=2048, k_ss=128, v=16,
             v_sb=16384, v_sh=2048, v_ss=128, out=16, o_sb=2048, B=4, Hq=16, Hkv=8, D=128, n_live=3, scale=0.088)
    a.update(kw)
    rc = _lib.lib().q3a_cp_attn_append(a["q"], a["q_sb"], a["kn"], a["kn_sb"], a["vn"], a["vn_sb"], a["k"],
                                       a["k_sb"], a["k_sh"], a["k_ss"], a["v"], a["v_sb"], a["v_sh"], a["v_ss"],
                                       a["out"], a["o_sb"], a["B"], a["Hq"], a["Hkv"], a["D"], a["n_live"],
                                       a["scale"], None)
    assert rc < 0 and frag in _lib.lib().q3a_last_error().decode()


@pytest.mark.parametrize("kw,frag", [
    (dict(qn=None), "null norm weight"), (dict(sin=None), "null norm weight"), (dict(cos=24), "16-byte aligned"),
    (dict(kn=None, ), "null norm weight"), (dict(k_new=None), "k_new"), (dict(n_live=0), "n_live"),
    (dict(Hq=8), "num_q_heads"), (dict(D=64), "head_dim"),
])
def test_cp_attn_append_rope_rejects_bad_arguments(kw, frag):
    a = dict(q=16, q_sb=4096, k_new=16, kn_sb=4096, v_new=16, vn_sb=4096, qn=16, kn=16, cos=16, sin=16, eps=1e-6,
             k=16, k_sb=16384, k_sh=2048, k_ss=128, v=16, v_sb=16384, v_sh=2048, v_ss=128, out=16, o_sb=2048, B=4,
             Hq=16, Hkv=8, D=128, n_live=3, scale=0.088)
    a.update(kw)
    rc = _lib.lib().q3a_cp_attn_append_rope(a["q"], a["q_sb"], a["k_new"], a["kn_sb"], a["v_new"], a["vn_sb"], a["qn"],
                                            a["kn"], a["cos"], a["sin"], a["eps"], a["k"], a["k_sb"], a["k_sh"],
                                            a["k_ss"], a["v"], a["v_sb"], a["v_sh"], a["v_ss"], a["out"], a["o_sb"],
                                            a["B"], a["Hq"], a["Hkv"], a["D"], a["n_live"], a["scale"], None)
    assert rc < 0 and frag in _lib.lib().q3a_last_error().decode()


def test_python_entry_points_refuse_cpu_tensors():
    q = torch.zeros(2, 1, 16, 128, dtype=torch.bfloat16)
    kc = torch.zeros(4, 16, 8, 128, dtype=torch.bfloat16)
    sl = torch.ones(2, dtype=torch.int32)
    bt = torch.zeros(2, 2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        q3attn.flash_attn_with_kvcache(q, kc, kc, cache_seqlens=sl, block_table=bt, softmax_scale=0.1, causal=True)
    with pytest.raises(RuntimeError, match="GPU"):
        q3attn.cp_attn(torch.zeros(2, 16, 128, dtype=torch.bfloat16), torch.zeros(2, 8, 16, 128, dtype=torch.bfloat16),
                       torch.zeros(2, 8, 16, 128, dtype=torch.bfloat16), 3, 0.1)
    with pytest.raises(RuntimeError, match="GPU"):
        q3attn.flash_attn_func(torch.zeros(2, 5, 16, 128, dtype=torch.bfloat16),
                               torch.zeros(2, 9, 8, 128, dtype=torch.bfloat16),
                               torch.zeros(2, 9, 8, 128, dtype=torch.bfloat16), causal=True)
    with pytest.raises(RuntimeError, match="GPU"):
        q3attn.cp_attn_append(torch.zeros(2, 16, 128, dtype=torch.bfloat16), torch.zeros(2, 8, 128, dtype=torch.bfloat16),
                              torch.zeros(2, 8, 128, dtype=torch.bfloat16), torch.zeros(2, 8, 16, 128, dtype=torch.bfloat16),
                              torch.zeros(2, 8, 16, 128, dtype=torch.bfloat16), 2, 0.1)


def test_unsupported_flash_attn_arguments_raise():
    q = torch.zeros(2, 1, 16, 128, dtype=torch.bfloat16)
    kc = torch.zeros(4, 16, 8, 128, dtype=torch.bfloat16)
    kw = dict(cache_seqlens=torch.ones(2, dtype=torch.int32), block_table=torch.zeros(2, 2, dtype=torch.int32))
    with pytest.raises(NotImplementedError):
        q3attn.flash_attn_with_kvcache(q, kc, kc, rotary_cos=q, **kw)
    with pytest.raises(NotImplementedError):
        q3attn.flash_attn_with_kvcache(q, kc, kc, window_size=(8, 0), **kw)
    with pytest.raises(RuntimeError, match="both k and v"):
        q3attn.flash_attn_with_kvcache(q, kc, kc, k=q, **kw)
    with pytest.raises(RuntimeError, match="GPU"):
        q3attn.flash_attn_with_kvcache(q, kc, kc, k=torch.zeros(2, 1, 8, 128, dtype=torch.bfloat16),
                                       v=torch.zeros(2, 1, 8, 128, dtype=torch.bfloat16), **kw)


@pytest.mark.parametrize("kw,frag", [
    (dict(kn=None), "k_new"), (dict(vn=None), "k_new"), (dict(kn=18), "aligned"), (dict(vn_sb=1030), "strides"),
    (dict(page=24), "page_size"), (dict(Hq=8), "num_q_heads"),
])
def test_paged_decode_append_rejects_bad_arguments(kw, frag):
    a = dict(q=16, q_sb=2048, q_sh=128, kn=16, kn_sb=1024, vn=16, vn_sb=4096, k=16, v=16, sp=16384, st=1024,
             sh=128, num_pages=8, page=16, seqlens=16, bt=16, bt_sb=4, max_pages=4, out=16, o_sb=2048, o_sh=128,
             ws=16, ws_bytes=1 << 30, B=2, Hq=16, Hkv=8, D=128, scale=0.088, split=0)
    a.update(kw)
    rc = _lib.lib().q3a_paged_decode_append(
        a["q"], a["q_sb"], a["q_sh"], a["kn"], a["kn_sb"], a["vn"], a["vn_sb"], a["k"], a["v"], a["sp"], a["st"],
        a["sh"], a["num_pages"], a["page"], a["seqlens"], a["bt"], a["bt_sb"], a["max_pages"], a["out"], a["o_sb"],
        a["o_sh"], a["ws"], a["ws_bytes"], a["B"], a["Hq"], a["Hkv"], a["D"], a["scale"], a["split"], None)
    assert rc < 0 and frag in _lib.lib().q3a_last_error().decode()


@pytest.mark.parametrize("kw,frag", [
    (dict(qn=None), "norm weight"), (dict(cs=None), "cos/sin"), (dict(cs=24), "16-byte aligned"),
    (dict(cs_sb=100), "16-byte aligned"), (dict(eps=-1.0), "eps"), (dict(split=64), "split_tokens <= 0"),
    (dict(B=65, max_pages=256, Hkv=16, Hq=32), "at most 8 KV heads"), (dict(kn=None), "k_new"),
    (dict(page=24), "page_size"),
])
def test_paged_decode_append_rope_rejects_bad_arguments(kw, frag):
    a = dict(q=16, q_sb=2048, q_sh=128, kn=16, kn_sb=1024, vn=16, vn_sb=4096, qn=16, knw=16, cs=16, cs_sb=128,
             eps=1e-6, k=16, v=16, sp=16384, st=1024, sh=128, num_pages=8, page=16, seqlens=16, bt=16, bt_sb=4,
             max_pages=4, out=16, o_sb=2048, o_sh=128, ws=16, ws_bytes=1 << 30, B=2, Hq=16, Hkv=8, D=128,
             scale=0.088, split=0)
    a.update(kw)
    rc = _lib.lib().q3a_paged_decode_append_rope(
        a["q"], a["q_sb"], a["q_sh"], a["kn"], a["kn_sb"], a["vn"], a["vn_sb"], a["qn"], a["knw"], a["cs"], a["cs"],
        a["cs_sb"], a["eps"], a["k"], a["v"], a["sp"], a["st"], a["sh"], a["num_pages"], a["page"], a["seqlens"],
        a["bt"], a["bt_sb"], a["max_pages"], a["out"], a["o_sb"], a["o_sh"], a["ws"], a["ws_bytes"], a["B"], a["Hq"],
        a["Hkv"], a["D"], a["scale"], a["split"], None)
    assert rc < 0 and frag in _lib.lib().q3a_last_error().decode(), _lib.lib().q3a_last_error().decode()


def test_paged_decode_append_rope_python_checks():
    """The torch op validates the norm weights and the cos/sin rows before calling the library."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        q = torch.empty(3, 16, 128, dtype=torch.bfloat16)
        kc = torch.empty(10, 16, 8, 128, dtype=torch.bfloat16)
        kv = torch.empty(3, 8, 128, dtype=torch.bfloat16)
        w = torch.empty(128, dtype=torch.bfloat16)
        cs = torch.empty(3, 1, 128, dtype=torch.bfloat16)
        o = torch.ops.q3attn.paged_decode_append_rope(q, kv, kv, w, w, cs, cs, kc, kc, torch.empty(3, dtype=torch.int32),
                                                      torch.empty(3, 4, dtype=torch.int32), 0.1, 1e-6)
        assert o.shape == (3, 16, 128) and o.dtype == torch.bfloat16
    q = torch.zeros(3, 16, 128, dtype=torch.bfloat16)
    kc = torch.zeros(10, 16, 8, 128, dtype=torch.bfloat16)
    kv = torch.zeros(3, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):   # CPU tensors are refused before any weight check
        q3attn.paged_decode_append_rope(q, kv, kv, torch.zeros(128, dtype=torch.bfloat16),
                                        torch.zeros(128, dtype=torch.bfloat16), torch.zeros(3, 128, dtype=torch.bfloat16),
                                        torch.zeros(3, 128, dtype=torch.bfloat16), kc, kc,
                                        torch.zeros(3, dtype=torch.int32), torch.zeros(3, 4, dtype=torch.int32), 0.1)


def test_fake_impl_traces_shapes():
    """The custom ops carry fake implementations, so torch.compile / export can trace through them
    without running the kernels."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        q = torch.empty(3, 16, 128, dtype=torch.bfloat16)
        kc = torch.empty(10, 16, 8, 128, dtype=torch.bfloat16)
        o = torch.ops.q3attn.paged_decode(q, kc, kc, torch.empty(3, dtype=torch.int32),
                                          torch.empty(3, 4, dtype=torch.int32), 0.1, 0)
        assert o.shape == (3, 16, 128) and o.dtype == torch.bfloat16
        kv = torch.empty(3, 8, 128, dtype=torch.bfloat16)
        o = torch.ops.q3attn.paged_decode_append(q, kv, kv, kc, kc, torch.empty(3, dtype=torch.int32),
                                                 torch.empty(3, 4, dtype=torch.int32), 0.1, 0)
        assert o.shape == (3, 16, 128)
        c = torch.ops.q3attn.cp_attn(q, torch.empty(3, 8, 16, 128, dtype=torch.bfloat16),
                                     torch.empty(3, 8, 16, 128, dtype=torch.bfloat16), 4, 0.1)
        assert c.shape == (3, 2048)
        p = torch.ops.q3attn.prefill_dense(torch.empty(2, 5, 16, 128, dtype=torch.bfloat16),
                                           torch.empty(2, 9, 8, 128, dtype=torch.bfloat16),
                                           torch.empty(2, 9, 8, 128, dtype=torch.bfloat16), 0.1, True)
        assert p.shape == (2, 5, 16, 128)
        kv = torch.empty(3, 8, 128, dtype=torch.bfloat16)
        c = torch.ops.q3attn.cp_attn_append(q, kv, kv, torch.empty(3, 8, 16, 128, dtype=torch.bfloat16),
                                            torch.empty(3, 8, 16, 128, dtype=torch.bfloat16), 4, 0.1)
        assert c.shape == (3, 2048)


@pytest.mark.parametrize("kw,frag", [
    (dict(D=64), "head_dim"), (dict(Hq=8), "num_q_heads"), (dict(q=None), "null pointer"), (dict(k=18), "aligned"),
    (dict(v=40), "aligned"), (dict(q_st=2050), "strides"), (dict(k_st=64), "token strides"),
    (dict(v_st=64), "token strides"), (dict(v_sh=3), "strides"), (dict(q_ss=-2048), "sequence strides"),
    (dict(v_ss=-8), "sequence strides"), (dict(o_ss=12), "sequence strides"), (dict(Lk=-1), "negative"),
    (dict(S=-1), "negative"),
])
def test_prefill_dense_rejects_bad_arguments(kw, frag):
    a = dict(q=16, q_ss=42 * 2048, q_st=2048, q_sh=128, k=16, k_ss=77 * 1024, k_st=1024, k_sh=128, v=16,
             v_ss=77 * 4096, v_st=4096, v_sh=128, out=16, o_ss=42 * 2048, o_st=2048, o_sh=128, S=8, Lq=42, Lk=77,
             Hq=16, Hkv=8, D=128, scale=0.088, causal=1)
    a.update(kw)
    rc = _lib.lib().q3a_prefill_dense(a["q"], a["q_ss"], a["q_st"], a["q_sh"], a["k"], a["k_ss"], a["k_st"],
                                      a["k_sh"], a["v"], a["v_ss"], a["v_st"], a["v_sh"], a["out"], a["o_ss"],
                                      a["o_st"], a["o_sh"], a["S"], a["Lq"], a["Lk"], a["Hq"], a["Hkv"], a["D"],
                                      a["scale"], a["causal"], None)
    assert rc < 0 and frag in _lib.lib().q3a_last_error().decode()


def test_prefill_dense_empty_is_a_noop():
    L = _lib.lib()
    assert L.q3a_prefill_dense(16, 0, 2048, 128, 16, 0, 1024, 128, 16, 0, 4096, 128, 16, 0, 2048, 128, 0, 42, 77, 16,
                               8, 128, 0.1, 1, None) == 0
    assert L.q3a_prefill_dense(16, 0, 2048, 128, 16, 0, 1024, 128, 16, 0, 4096, 128, 16, 0, 2048, 128, 8, 0, 77, 16,
                               8, 128, 0.1, 1, None) == 0


def _prefill(**kw):
    """The talker's own prefill layout (engine/talker.py:157-169): q [T,16,128] and k [T,8,128] fresh tensors, v a
    view of the [T, 4096] qkv projection (token stride 4096)."""
    a = dict(q=16, q_st=2048, q_sh=128, cu_q=16, k=16, k_sp=0, k_st=1024, k_sh=128, v=16, v_sp=0, v_st=4096,
             v_sh=128, num_pages=0, page=0, bt=None, bt_sb=0, max_pages=0, cu_k=16, out=16, o_st=2048, o_sh=128,
             n=4, max_q=400, Hq=16, Hkv=8, D=128, scale=0.088, causal=1)
    a.update(kw)
    return _lib.lib().q3a_prefill(a["q"], a["q_st"], a["q_sh"], a["cu_q"], a["k"], a["k_sp"], a["k_st"], a["k_sh"],
                                  a["v"], a["v_sp"], a["v_st"], a["v_sh"], a["num_pages"], a["page"], a["bt"],
                                  a["bt_sb"], a["max_pages"], a["cu_k"], a["out"], a["o_st"], a["o_sh"], a["n"],
                                  a["max_q"], a["Hq"], a["Hkv"], a["D"], a["scale"], a["causal"], None)


@pytest.mark.parametrize("kw,frag", [
    (dict(D=64), "head_dim"), (dict(cu_q=None), "null pointer"), (dict(v=None), "null pointer"),
    (dict(v=8), "aligned"), (dict(v_st=4100), "strides"), (dict(k_st=64), "token strides"),
    (dict(v_st=(1 << 26) + 8), "token strides"), (dict(n=-1), "negative"),
    (dict(bt=16, page=16, num_pages=0, max_pages=4), "paged K/V"),
    (dict(bt=16, page=48, num_pages=8, max_pages=4, k_sp=16384, v_sp=16384), "power of two"),
    (dict(bt=16, page=16, num_pages=8, max_pages=4, k_sp=16384, v_sp=16380), "page strides"),
])
def test_prefill_rejects_bad_arguments(kw, frag):
    assert _prefill(**kw) < 0
    assert frag in _lib.lib().q3a_last_error().decode()


def _prefill_append(**kw):
    a = dict(q=16, q_st=2048, q_sh=128, cu_q=16, k=16, k_st=1024, k_sh=128, v=16, v_st=4096, v_sh=128, cu_k=16,
             kc=16, vc=16, c_sp=16384, c_st=1024, c_sh=128, num_pages=8, page=16, bt=16, bt_sb=4, max_pages=4,
             out=16, o_st=2048, o_sh=128, n=2, max_q=40, Hq=16, Hkv=8, D=128, scale=0.088, causal=1)
    a.update(kw)
    return _lib.lib().q3a_prefill_append(a["q"], a["q_st"], a["q_sh"], a["cu_q"], a["k"], a["k_st"], a["k_sh"],
                                         a["v"], a["v_st"], a["v_sh"], a["cu_k"], a["kc"], a["vc"], a["c_sp"],
                                         a["c_st"], a["c_sh"], a["num_pages"], a["page"], a["bt"], a["bt_sb"],
                                         a["max_pages"], a["out"], a["o_st"], a["o_sh"], a["n"], a["max_q"], a["Hq"],
                                         a["Hkv"], a["D"], a["scale"], a["causal"], None)


@pytest.mark.parametrize("kw,frag", [
    (dict(kc=None), "null pointer"), (dict(bt=None), "null pointer"), (dict(cu_k=None), "null pointer"),
    (dict(page=48), "power of two"), (dict(page=8), "power of two"), (dict(num_pages=0), "num_pages"),
    (dict(vc=8), "aligned"), (dict(c_st=64), "cache strides"), (dict(c_sp=1024), "cache strides"),
    (dict(c_sh=-128), "cache strides"), (dict(D=64), "head_dim"), (dict(v_st=4100), "strides"),
])
def test_prefill_append_rejects_bad_arguments(kw, frag):
    assert _prefill_append(**kw) < 0
    assert frag in _lib.lib().q3a_last_error().decode()


def test_prefill_append_empty_is_a_noop():
    assert _prefill_append(n=0) == 0 and _prefill_append(max_q=0) == 0


def _prefill_dense_append(**kw):
    """The admission shape (engine/arrivals.py:144-148): S = 8, R = 42 over n = 77 keys, fake aligned pointers."""
    a = dict(q=16, q_ss=42 * 2048, q_st=2048, q_sh=128, k=16, k_ss=77 * 1024, k_st=1024, k_sh=128,
             v=16, v_ss=77 * 1024, v_st=1024, v_sh=128, kc=16, vc=16, c_sp=16384, c_st=1024, c_sh=128,
             num_pages=64, page=16, bt=16, bt_sb=8, max_pages=8, first=0, out=16, o_ss=42 * 2048, o_st=2048,
             o_sh=128, S=8, R=42, n=77, Hq=16, Hkv=8, D=128, scale=0.088, causal=1)
    a.update(kw)
    return _lib.lib().q3a_prefill_dense_append(
        a["q"], a["q_ss"], a["q_st"], a["q_sh"], a["k"], a["k_ss"], a["k_st"], a["k_sh"], a["v"], a["v_ss"],
        a["v_st"], a["v_sh"], a["kc"], a["vc"], a["c_sp"], a["c_st"], a["c_sh"], a["num_pages"], a["page"], a["bt"],
        a["bt_sb"], a["max_pages"], a["first"], a["out"], a["o_ss"], a["o_st"], a["o_sh"], a["S"], a["R"], a["n"],
        a["Hq"], a["Hkv"], a["D"], a["scale"], a["causal"], None)


@pytest.mark.parametrize("kw,frag", [
    (dict(kc=None), "null pointer"), (dict(bt=None), "null pointer"), (dict(k=None), "null pointer"),
    (dict(page=48), "power of two"), (dict(num_pages=0), "num_pages"), (dict(max_pages=0), "num_pages"),
    (dict(vc=8), "aligned"), (dict(c_st=64), "cache strides"), (dict(c_sp=1024), "cache strides"),
    (dict(first=-1), "first_row"), (dict(first=36), "first_row"), (dict(n=40, first=1), "first_row"),
    (dict(D=64), "head_dim"), (dict(k_ss=-8), "sequence strides"), (dict(S=-1), "negative"),
])
def test_prefill_dense_append_rejects_bad_arguments(kw, frag):
    assert _prefill_dense_append(**kw) < 0
    assert frag in _lib.lib().q3a_last_error().decode()


def _dense_rope(**kw):
    """The admission shape (S = 8, R = 42 new tokens after a 35-token prefix), fake aligned pointers; q/k/v as views
    of a [S, R, 4096] qkv projection."""
    a = dict(q=16, q_ss=42 * 4096, q_st=4096, q_sh=128, k=16, k_ss=42 * 4096, k_st=4096, k_sh=128,
             v=16, v_ss=42 * 4096, v_st=4096, v_sh=128, pk=16, pk_ss=35 * 1024, pk_st=1024, pk_sh=128,
             pv=16, pv_ss=35 * 1024, pv_st=1024, pv_sh=128, pidx=None, npre=8, qn=16, kn=16, cos=16, sin=16,
             rope_st=128, eps=1e-6, kc=16, vc=16, c_sp=16384, c_st=1024, c_sh=128, num_pages=64, page=16, bt=16,
             bt_sb=8, max_pages=8, first=0, out=16, o_ss=42 * 2048, o_st=2048, o_sh=128, ws=16, ws_bytes=1 << 30,
             S=8, R=42, P=35, Hq=16, Hkv=8, D=128, scale=0.088, causal=1)
    a.update(kw)
    return _lib.lib().q3a_prefill_dense_append_rope(
        a["q"], a["q_ss"], a["q_st"], a["q_sh"], a["k"], a["k_ss"], a["k_st"], a["k_sh"], a["v"], a["v_ss"], a["v_st"],
        a["v_sh"], a["pk"], a["pk_ss"], a["pk_st"], a["pk_sh"], a["pv"], a["pv_ss"], a["pv_st"], a["pv_sh"], a["pidx"],
        a["npre"], a["qn"], a["kn"], a["cos"], a["sin"], a["rope_st"], a["eps"], a["kc"], a["vc"], a["c_sp"],
        a["c_st"], a["c_sh"], a["num_pages"], a["page"], a["bt"], a["bt_sb"], a["max_pages"], a["first"], a["out"],
        a["o_ss"], a["o_st"], a["o_sh"], a["ws"], a["ws_bytes"], a["S"], a["R"], a["P"], a["Hq"], a["Hkv"], a["D"],
        a["scale"], a["causal"], None)


@pytest.mark.parametrize("kw,frag", [
    (dict(qn=None), "null pointer"), (dict(pk=None), "null pointer"), (dict(ws=None), "null pointer"),
    (dict(kc=None), "null pointer"), (dict(cos=8), "aligned"), (dict(ws=8), "aligned"), (dict(q_st=4100), "strides"),
    (dict(rope_st=-128), "strides"), (dict(first=36), "first_row"), (dict(first=-1), "first_row"),
    (dict(ws_bytes=1024), "workspace"), (dict(D=64), "head_dim"), (dict(Hq=12), "num_q_heads"),
    (dict(Hq=12, Hkv=6), "multiple of 4"), (dict(npre=0), "num_prefixes"), (dict(page=48), "power of two"),
    (dict(P=-1), "negative"),
    # the prefix bank's token strides bound one 32-bit buffer extent per 16-row group, as k and v's do
    (dict(pk_st=(1 << 26) + 8), "prefix token strides"), (dict(pv_st=(1 << 27)), "prefix token strides"),
    (dict(pk_st=64), "prefix token strides"),
])
def test_prefill_dense_append_rope_rejects_bad_arguments(kw, frag):
    assert _dense_rope(**kw) < 0
    assert frag in _lib.lib().q3a_last_error().decode()


def test_prefill_dense_append_rope_workspace_and_noop():
    L = _lib.lib()
    # q [8, 42, 16, 128] + K and V [8, 77, 8, 128] in bf16, each part rounded up to 256 B
    assert L.q3a_prefill_dense_append_rope_workspace_bytes(8, 42, 35, 16, 8, 128) == 8 * 42 * 16 * 256 + 2 * 8 * 77 * 8 * 256
    assert L.q3a_prefill_dense_append_rope_workspace_bytes(0, 42, 35, 16, 8, 128) == 0
    assert _dense_rope(S=0) == 0 and _dense_rope(R=0) == 0


def _prompt_rope(**kw):
    """The prompt-step shape (32 sequences, 8,800 tokens), q/k/v as views of a [T, 4096] qkv projection."""
    a = dict(q=16, q_st=4096, q_sh=128, k=16, k_st=4096, k_sh=128, v=16, v_st=4096, v_sh=128, qn=16, kn=16, cos=16,
             sin=16, rope_st=128, eps=1e-6, cu=16, kc=16, vc=16, c_sp=16384, c_st=1024, c_sh=128, num_pages=1024,
             page=16, bt=16, bt_sb=32, max_pages=32, out=16, o_st=2048, o_sh=128, ws=16, ws_bytes=1 << 30, n=32,
             T=8800, L=400, Hq=16, Hkv=8, D=128, scale=0.088, causal=1)
    a.update(kw)
    return _lib.lib().q3a_prefill_append_rope(
        a["q"], a["q_st"], a["q_sh"], a["k"], a["k_st"], a["k_sh"], a["v"], a["v_st"], a["v_sh"], a["qn"], a["kn"],
        a["cos"], a["sin"], a["rope_st"], a["eps"], a["cu"], a["kc"], a["vc"], a["c_sp"], a["c_st"], a["c_sh"],
        a["num_pages"], a["page"], a["bt"], a["bt_sb"], a["max_pages"], a["out"], a["o_st"], a["o_sh"], a["ws"],
        a["ws_bytes"], a["n"], a["T"], a["L"], a["Hq"], a["Hkv"], a["D"], a["scale"], a["causal"], None)


@pytest.mark.parametrize("kw,frag", [
    (dict(kn=None), "null pointer"), (dict(cu=None), "null pointer"), (dict(ws=None, causal=0), "null pointer"),
    (dict(bt=None), "null pointer"), (dict(sin=24), "aligned"), (dict(k_st=4100), "strides"),
    (dict(ws_bytes=4096, causal=0), "workspace"), (dict(ws=24, causal=0), "aligned"), (dict(out=24), "aligned"),
    (dict(o_st=2052), "strides"), (dict(v_st=64), "token strides"), (dict(D=256), "head_dim"),
    (dict(Hq=8), "num_q_heads"),
    (dict(Hq=12, Hkv=6), "multiple of 4"), (dict(page=24), "power of two"), (dict(T=-5), "negative"),
])
def test_prefill_append_rope_rejects_bad_arguments(kw, frag):
    assert _prompt_rope(**kw) < 0
    assert frag in _lib.lib().q3a_last_error().decode()


def test_prefill_append_rope_workspace_and_noop():
    L = _lib.lib()
    assert L.q3a_prefill_append_rope_workspace_bytes(8800, 16, 8, 128) == 8800 * 16 * 256 + 8800 * 8 * 256
    assert L.q3a_prefill_append_rope_workspace_bytes(0, 16, 8, 128) == 0
    assert _prompt_rope(n=0) == 0 and _prompt_rope(T=0) == 0 and _prompt_rope(L=0) == 0


def test_prefill_dense_append_empty_is_a_noop():
    """Nothing to compute or write: no device pointer is touched (these are fake addresses)."""
    assert _prefill_dense_append(S=0) == 0 and _prefill_dense_append(R=0, first=0) == 0


def test_prefill_empty_is_a_noop():
    assert _prefill(n=0) == 0 and _prefill(max_q=0) == 0


def test_prefill_accepts_the_reference_kv_layout_on_the_host_side():
    """The equal-stride requirement is gone from the Python op: only shape and the contiguous head dim are checked
    before any device work, so the error a CPU tensor raises is the device one."""
    T = 10
    qkv = torch.zeros(T, 4096, dtype=torch.bfloat16)
    q = torch.zeros(T, 16, 128, dtype=torch.bfloat16)
    k = torch.zeros(T, 8, 128, dtype=torch.bfloat16)
    v = qkv[:, 3072:].view(T, 8, 128)
    assert k.stride() != v.stride()
    cu = torch.tensor([0, 4, T], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        q3attn.flash_attn_varlen_func(q, k, v, cu, cu, 6, 6, softmax_scale=0.1, causal=True)
