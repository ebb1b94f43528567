"""The C ABI library loads without a GPU, exports every entry point that
include/gdn.h declares, and rejects bad arguments before launching anything
(negative codes + a thread-local message).  No compute call needs a device."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    from avelang_amd import _native
    return _native.lib()


def _declared(headers=("gdn.h", "gdn_layer.h")):
    names = set()
    for h in headers:
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(gdn_\w+)\s*\(", text))
    return sorted(names)


def test_header_declares_expected_entry_points():
    assert _declared(("gdn.h",)) == ["gdn_abi_version", "gdn_chunk_bwd",
                                     "gdn_chunk_bwd_workspace_bytes", "gdn_chunk_fwd",
                                     "gdn_chunk_fwd_noalloc", "gdn_chunk_fwd_save",
                                     "gdn_chunk_workspace_bytes", "gdn_cu_seqlens_check",
                                     "gdn_last_error", "gdn_recurrent_fwd"]
    assert _declared(("gdn_layer.h",)) == [
        "gdn_causal_conv1d_fwd", "gdn_causal_conv1d_update", "gdn_chunk_fwd_gating",
        "gdn_gating_bwd", "gdn_gating_bwd_workspace_bytes",
        "gdn_gating_fwd", "gdn_l2norm_fwd", "gdn_recurrent_fwd_gating",
        "gdn_recurrent_fwd_indexed", "gdn_recurrent_fwd_spec", "gdn_rmsnorm_gated_fwd"]


def test_every_declared_symbol_is_exported(lib):
    from avelang_amd import _native
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_native.EXPORTS) == set(_declared())
    assert lib.gdn_abi_version() == 101


def _rec(lib, **kw):
    p = dict(q=1 << 20, k=2 << 20, v=3 << 20, g=4 << 20, beta=5 << 20, h0=None, ht=None,
             o=6 << 20, cu=None,
             B=1, T=4, Hqk=2, Hv=4, K=128, V=128, N=1, scale=0.1, l2=0, stream=None)
    p.update(kw)
    return lib.gdn_recurrent_fwd(p["q"], p["k"], p["v"], p["g"], p["beta"], p["h0"], p["ht"],
                                 p["o"], p["cu"], p["B"], p["T"], p["Hqk"], p["Hv"], p["K"],
                                 p["V"], p["N"], p["scale"], p["l2"], p["stream"])


def _chunk(lib, ws=None, wsb=0, **kw):
    p = dict(q=1 << 20, k=2 << 20, v=3 << 20, g=4 << 20, beta=5 << 20, h0=None, ht=None,
             o=6 << 20, cu=None,
             B=1, T=4, Hqk=2, Hv=4, K=128, V=128, N=1, scale=0.1, l2=0, stream=None)
    p.update(kw)
    return lib.gdn_chunk_fwd(p["q"], p["k"], p["v"], p["g"], p["beta"], p["h0"], p["ht"],
                             p["o"], p["cu"], p["B"], p["T"], p["Hqk"], p["Hv"], p["K"],
                             p["V"], p["N"], p["scale"], p["l2"], ws, wsb, p["stream"])


@pytest.mark.parametrize("fn", [_rec, _chunk])
@pytest.mark.parametrize("kw,code,msg", [
    (dict(Hv=3), -2, "multiple of Hqk"),
    (dict(K=96), -2, "unsupported head sizes"),
    (dict(V=32), -2, "unsupported head sizes"),
    (dict(T=-1), -2, "non-negative"),
    (dict(N=2), -3, "N must equal B"),
    (dict(cu=8, B=2, N=2), -3, "B == 1"),
    (dict(q=None), -1, "non-NULL"),
    (dict(o=None), -1, "non-NULL"),
    (dict(h0=7 << 20, ht=(7 << 20) + 64), -5, "must equal h0"),
    (dict(o=1 << 20), -5, "must not overlap"),
])
def test_argument_errors(lib, fn, kw, code, msg):
    from avelang_amd import _native
    rc = fn(lib, **kw)
    assert rc == code
    assert msg in _native.last_error()


def _bwd(lib, ws=None, wsb=0, **kw):
    M = 1 << 20
    p = dict(q=1 * M, k=2 * M, v=3 * M, g=4 * M, beta=5 * M, h0=None, do=6 * M, dht=None,
             dq=7 * M, dk=8 * M, dv=9 * M, dg=10 * M, db=11 * M, dh0=None, cu=None,
             B=1, T=4, Hqk=2, Hv=4, K=128, V=128, N=1, scale=0.1, l2=0, saved=0, stream=None)
    p.update(kw)
    return lib.gdn_chunk_bwd(p["q"], p["k"], p["v"], p["g"], p["beta"], p["h0"], p["do"],
                             p["dht"], p["dq"], p["dk"], p["dv"], p["dg"], p["db"], p["dh0"],
                             p["cu"], p["B"], p["T"], p["Hqk"], p["Hv"], p["K"], p["V"], p["N"],
                             p["scale"], p["l2"], p["saved"], ws, wsb, p["stream"])


@pytest.mark.parametrize("kw,code,msg", [
    (dict(Hv=3), -2, "multiple of Hqk"),
    (dict(dq=None), -1, "must be non-NULL"),
    (dict(dbeta=None, db=None), -1, "must be non-NULL"),
    (dict(dq=(1 << 20) + 64), -5, "overlaps an input"),
    (dict(dv=(6 << 20) + 128), -5, "overlaps an input"),
    (dict(dk=(7 << 20) + 32), -5, "two gradient buffers overlap"),
    (dict(do=2 << 20), -5, "must not overlap"),
])
def test_bwd_argument_errors(lib, kw, code, msg):
    from avelang_amd import _native
    kw.pop("dbeta", None)
    assert _bwd(lib, **kw) == code
    assert msg in _native.last_error()


def test_bwd_workspace_checked_before_launch(lib):
    from avelang_amd import _native
    need = lib.gdn_chunk_bwd_workspace_bytes(1, 4, 2, 4, 128, 128, 1, 0, 0)
    fwd = lib.gdn_chunk_workspace_bytes(1, 4, 2, 4, 128, 128, 1, 0, 0)
    assert need > fwd > 0
    assert _bwd(lib) == -4
    assert "workspace needs" in _native.last_error()
    assert _bwd(lib, ws=64 << 20, wsb=need - 1) == -4
    # the training forward takes the backward's (larger) workspace
    rc = lib.gdn_chunk_fwd_save(1 << 20, 2 << 20, 3 << 20, 4 << 20, 5 << 20, None, None, 6 << 20,
                                None, 1, 4, 2, 4, 128, 128, 1, 0.1, 0, 64 << 20, fwd, None)
    assert rc == -4 and "gdn_chunk_fwd_save" in _native.last_error()


def test_chunk_workspace_checked_before_launch(lib):
    from avelang_amd import _native
    need = lib.gdn_chunk_workspace_bytes(1, 4, 2, 4, 128, 128, 1, 0, 0)
    assert need > 0
    assert _chunk(lib, ws=None, wsb=0) == -4
    assert "workspace needs" in _native.last_error()
    assert _chunk(lib, ws=8 << 20, wsb=need - 1) == -4


def test_workspace_bytes_grow_with_problem(lib):
    f = lib.gdn_chunk_workspace_bytes
    a = f(1, 8192, 16, 32, 128, 128, 1, 0, 0)
    b = f(1, 16384, 16, 32, 128, 128, 1, 0, 0)
    c = f(1, 8192, 16, 32, 128, 128, 64, 1, 0)
    d = f(1, 8192, 16, 32, 128, 128, 1, 0, 1)
    assert 0 < a < b and c > a
    # per (chunk, v-head): 64 gate floats (G) + 6 KiB Tb + 6 KiB P fragments;
    # a forward without l2norm whose chains do not fill the GPU twice over
    # reads K and Q from the caller's rows, so no per-(chunk, qk-head) copies
    copies = 128 * 16 * (16384 + 16384)   # fp16 K block (16 KiB) + Q fragments (16 KiB)
    assert 128 * 32 * (256 + 6144 + 6144) <= a < 128 * 32 * (256 + 6144 + 6144) + copies
    # in-kernel l2norm: the chain reads the prep kernel's normalised fp16 copies
    assert d >= a + copies
    # the backward's workspace keeps the normalised rows with l2norm
    bw = lib.gdn_chunk_bwd_workspace_bytes
    assert bw(1, 8192, 16, 32, 128, 128, 1, 0, 1) > bw(1, 8192, 16, 32, 128, 128, 1, 0, 0)


def test_empty_problem_is_a_noop(lib):
    assert _rec(lib, T=0, q=None, k=None, v=None, g=None, beta=None, o=None) == 0
    assert _chunk(lib, T=0, B=0, N=0, q=None, k=None, v=None, g=None, beta=None, o=None) == 0


def test_last_error_is_thread_local(lib):
    import threading
    from avelang_amd import _native
    assert _rec(lib, Hv=3) == -2
    seen = {}

    def other():
        assert _rec(lib, K=96) == -2
        seen["msg"] = _native.last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert "K=96" in seen["msg"]
    assert "multiple of Hqk" in _native.last_error()


# ------------------------------------------------------- layer operators ----
def _conv(lib, **kw):
    p = dict(x=1 << 20, w=2 << 20, bias=None, sq=None, init=None, fin=None, out=3 << 20,
             B=1, D=16, T=8, W=4, xs=(128, 1, 16), os_=(128, 1, 16), silu=1, dt=1, wdt=1)
    p.update(kw)
    return lib.gdn_causal_conv1d_fwd(p["x"], p["w"], p["bias"], p["sq"], p["init"], p["fin"],
                                     p["out"], p["B"], p["D"], p["T"], p["W"], *p["xs"],
                                     *p["os_"], p["silu"], p["dt"], p["wdt"], None)


def _convu(lib, **kw):
    p = dict(x=1 << 20, st=2 << 20, w=3 << 20, bias=None, idx=None, out=4 << 20,
             B=2, D=16, L=1, W=4, S=3, slots=2, xs=(16, 1, 16), os_=(16, 1, 16),
             silu=1, dt=1, wdt=1)
    p.update(kw)
    return lib.gdn_causal_conv1d_update(p["x"], p["st"], p["w"], p["bias"], p["idx"],
                                        p["out"], p["B"], p["D"], p["L"], p["W"], p["S"],
                                        p["slots"], *p["xs"], *p["os_"], p["silu"], p["dt"],
                                        p["wdt"], None)


def _reci(lib, **kw):
    p = dict(q=1 << 20, k=2 << 20, v=3 << 20, g=4 << 20, beta=5 << 20, h0=7 << 20, ht=7 << 20,
             o=6 << 20, cu=None, idx=8 << 20, B=2, T=1, Hqk=2, Hv=4, K=128, V=128, N=2,
             slots=4)
    p.update(kw)
    return lib.gdn_recurrent_fwd_indexed(p["q"], p["k"], p["v"], p["g"], p["beta"], p["h0"],
                                         p["ht"], p["o"], p["cu"], p["idx"], p["B"], p["T"],
                                         p["Hqk"], p["Hv"], p["K"], p["V"], p["N"], p["slots"],
                                         0.1, 0, None)


def _recs(lib, **kw):
    p = dict(q=1 << 20, k=2 << 20, v=3 << 20, g=4 << 20, beta=5 << 20, pool=7 << 20,
             o=6 << 20, cu=None, idx=8 << 20, stride=4, acc=None, B=2, T=4, Hqk=2, Hv=4,
             K=128, V=128, N=2, slots=8)
    p.update(kw)
    return lib.gdn_recurrent_fwd_spec(p["q"], p["k"], p["v"], p["g"], p["beta"], p["pool"],
                                      p["o"], p["cu"], p["idx"], p["stride"], p["acc"], p["B"],
                                      p["T"], p["Hqk"], p["Hv"], p["K"], p["V"], p["N"],
                                      p["slots"], 0.1, 0, None)


def _gbwd(lib, **kw):
    """gdn_gating_bwd with fake (never dereferenced) pointers; rows 8, H 4."""
    p = dict(A=1 << 20, a=2 << 20, b=3 << 20, dtb=4 << 20, dg=5 << 20, dbeta=6 << 20,
             dA=7 << 20, da=8 << 20, db=9 << 20, ddt=10 << 20, rows=8, H=4, adt=1, bdt=1,
             pdt=0, spb=1.0, spt=20.0, ws=11 << 20, wsb=1 << 16)
    p.update(kw)
    return lib.gdn_gating_bwd(p["A"], p["a"], p["b"], p["dtb"], p["dg"], p["dbeta"], p["dA"],
                              p["da"], p["db"], p["ddt"], p["rows"], p["H"], p["adt"],
                              p["bdt"], p["pdt"], p["spb"], p["spt"], p["ws"], p["wsb"], None)


def test_gating_bwd_workspace_bytes(lib):
    # one (ddt_bias, dA_log) fp32 pair per head and block of 64 rows; at most
    # 1024 blocks (longer inputs take more rows per block)
    assert lib.gdn_gating_bwd_workspace_bytes(0, 32) == 0
    assert lib.gdn_gating_bwd_workspace_bytes(1, 32) == 32 * 8
    assert lib.gdn_gating_bwd_workspace_bytes(8192, 32) == 128 * 32 * 8
    assert lib.gdn_gating_bwd_workspace_bytes(1 << 20, 32) == 1024 * 32 * 8
    assert lib.gdn_gating_bwd_workspace_bytes((1 << 20) + 1, 4) <= 1025 * 4 * 8
    assert lib.gdn_gating_bwd_workspace_bytes(-1, 4) == 0


@pytest.mark.parametrize("call,code,msg", [
    (lambda l: _recs(l, stride=0), -2, "index_stride must be > 0"),
    (lambda l: _recs(l, T=5), -2, "exceeds index_stride"),
    (lambda l: _recs(l, idx=None), -1, "state_indices"),
    (lambda l: _recs(l, pool=None), -1, "pool"),
    (lambda l: _recs(l, slots=-1), -2, "num_slots"),
    (lambda l: _recs(l, K=96), -2, "unsupported head sizes"),
    (lambda l: l.gdn_gating_fwd(1 << 20, 2 << 20, 3 << 20, 4 << 20, 5 << 20, 6 << 20, 8, 0,
                                1, 1, 0, 1.0, 20.0, None), -2, "H > 0"),
    (lambda l: l.gdn_gating_fwd(1 << 20, 2 << 20, 3 << 20, 4 << 20, 5 << 20, 6 << 20, 8, 4,
                                7, 1, 0, 1.0, 20.0, None), -2, "dtype"),
    (lambda l: l.gdn_gating_fwd(1 << 20, 2 << 20, 3 << 20, 4 << 20, 5 << 20, 6 << 20, 8, 4,
                                1, 1, 0, 0.0, 20.0, None), -2, "softplus beta"),
    (lambda l: l.gdn_gating_fwd(None, 2 << 20, 3 << 20, 4 << 20, 5 << 20, 6 << 20, 8, 4,
                                1, 1, 0, 1.0, 20.0, None), -1, "non-NULL"),
    (lambda l: _gbwd(l, H=0), -2, "0 < H <= 256"),
    (lambda l: _gbwd(l, H=257), -2, "0 < H <= 256"),
    (lambda l: _gbwd(l, adt=5), -2, "dtype"),
    (lambda l: _gbwd(l, spb=0.0), -2, "softplus beta"),
    (lambda l: _gbwd(l, dg=None), -1, "non-NULL"),
    (lambda l: _gbwd(l, db=None), -1, "go together"),
    (lambda l: _gbwd(l, b=None), -1, "need b"),
    (lambda l: _gbwd(l, ws=None), -4, "workspace"),
    (lambda l: _gbwd(l, wsb=8), -4, "workspace"),
    (lambda l: l.gdn_l2norm_fwd(1 << 20, 2 << 20, 8, 96, 1e-6, 1, None), -2, "64, 128 or 256"),
    (lambda l: l.gdn_l2norm_fwd(None, 2 << 20, 8, 128, 1e-6, 1, None), -1, "non-NULL"),
    (lambda l: l.gdn_rmsnorm_gated_fwd(1 << 20, 2 << 20, 3 << 20, 4 << 20, 8, 100, 1e-6, 1, 1,
                                       None), -2, "64, 128 or 256"),
    (lambda l: l.gdn_rmsnorm_gated_fwd(1 << 20, None, 3 << 20, 4 << 20, 8, 128, 1e-6, 1, 1,
                                       None), -1, "non-NULL"),
    (lambda l: _conv(l, W=5), -2, "W must be"),
    (lambda l: _conv(l, dt=9), -2, "dtype"),
    (lambda l: _conv(l, sq=5 << 20, init=6 << 20), -2, "cannot be combined"),
    (lambda l: _conv(l, x=None), -1, "non-NULL"),
    (lambda l: _conv(l, out=1 << 20), -5, "alias"),
    (lambda l: _conv(l, xs=(128, -1, 16)), -2, "strides"),
    (lambda l: _convu(l, S=2), -2, "state length"),
    (lambda l: _convu(l, S=9), -2, "state length"),
    (lambda l: _convu(l, L=65), -2, "tokens per row"),
    (lambda l: _convu(l, slots=1), -2, "num_slots must be >= B"),
    (lambda l: _convu(l, st=None), -1, "non-NULL"),
    (lambda l: _reci(l, idx=None), -1, "state_indices"),
    (lambda l: _reci(l, ht=(7 << 20) + 64), -5, "must equal h0"),
    (lambda l: _reci(l, slots=-1), -2, "num_slots"),
    (lambda l: _reci(l, K=96), -2, "unsupported head sizes"),
])
def test_layer_argument_errors(lib, call, code, msg):
    from avelang_amd import _native
    rc = call(lib)
    assert rc == code, _native.last_error()
    assert msg in _native.last_error()


def test_layer_empty_problems_launch_nothing(lib):
    # zero-sized problems return before touching the (fake) pointers or a device
    assert lib.gdn_gating_fwd(1 << 20, 2 << 20, 3 << 20, 4 << 20, 5 << 20, 6 << 20, 0, 4,
                              1, 1, 0, 1.0, 20.0, None) == 0
    assert lib.gdn_l2norm_fwd(1 << 20, 2 << 20, 0, 128, 1e-6, 1, None) == 0
    assert _gbwd(lib, rows=0, dA=None, ddt=None, ws=None, wsb=0) == 0
    assert lib.gdn_rmsnorm_gated_fwd(1 << 20, 2 << 20, 3 << 20, 4 << 20, 0, 128, 1e-6, 1, 1,
                                     None) == 0
    assert _conv(lib, B=0) == 0
    assert _convu(lib, B=0) == 0
    assert _reci(lib, N=0, B=0) == 0
    assert _recs(lib, N=0, B=0) == 0


@pytest.mark.parametrize("cu, total, msg", [
    ([0, 3, 3, 10], 10, None),
    ([0], 0, None),                                  # N = 0
    ([0, 0, 0], 0, None),                            # empty sequences only
    ([1, 3, 10], 10, "cu_seqlens[0] must be 0"),
    ([0, 5, 4, 10], 10, "non-decreasing"),
    ([0, 3, 9], 10, "must equal the packed token count"),
    ([0, 3, 11], 10, "must equal the packed token count"),
])
def test_cu_seqlens_contract_host_check(lib, cu, total, msg):
    """gdn_cu_seqlens_check: the contract the chunked kernels check on the device."""
    arr = (ctypes.c_int32 * len(cu))(*cu)
    rc = lib.gdn_cu_seqlens_check(arr, len(cu) - 1, total)
    if msg is None:
        assert rc == 0
    else:
        assert rc == -3 and msg in lib.gdn_last_error().decode()


def test_cu_seqlens_check_arguments(lib):
    assert lib.gdn_cu_seqlens_check(None, 1, 4) == -1
    arr = (ctypes.c_int32 * 2)(0, 4)
    assert lib.gdn_cu_seqlens_check(arr, -1, 4) == -2


def test_noalloc_scratch_limit_checked_before_launch(lib):
    """gdn_chunk_fwd_noalloc rejects a problem over its 32 MiB scratch first."""
    need = lib.gdn_chunk_workspace_bytes(1, 8192, 16, 32, 128, 128, 1, 0, 0)
    assert need > (32 << 20)
    fake = [1 << 28, 2 << 28, 3 << 28, 4 << 28, 5 << 28, None, None, 6 << 28, None]
    assert lib.gdn_chunk_fwd_noalloc(*fake, 1, 8192, 16, 32, 128, 128, 1, 0.1, 0, None) == -4
    assert "scratch" in lib.gdn_last_error().decode()
    assert lib.gdn_chunk_fwd_noalloc(None, *fake[1:], 1, 64, 2, 4, 128, 128, 1, 0.1, 0, None) == -1


def test_fused_gating_argument_errors(lib):
    """The *_gating entry points check the gating arguments before launching."""
    P = [1 << 28, 2 << 28, 3 << 28]                       # q, k, v
    G = [4 << 28, 5 << 28, 6 << 28, 7 << 28]              # A_log, a, b, dt_bias
    tail = [None, None, 8 << 28, None, 1, 64, 2, 4, 128, 128, 1, 0.1, 0]
    ws = [9 << 28, 1 << 30, None]
    assert lib.gdn_chunk_fwd_gating(*P, *G, 7, 1, 0, 1.0, 20.0, *tail, *ws) == -2
    assert "dtype" in lib.gdn_last_error().decode()
    assert lib.gdn_chunk_fwd_gating(*P, *G, 1, 1, 0, 0.0, 20.0, *tail, *ws) == -2
    assert lib.gdn_chunk_fwd_gating(*P, None, *G[1:], 1, 1, 0, 1.0, 20.0, *tail, *ws) == -1
    assert lib.gdn_chunk_fwd_gating(*P, G[0], None, *G[2:], 1, 1, 0, 1.0, 20.0, *tail, *ws) == -1
    rtail = [None, None, 8 << 28, None, None, 1, 4, 2, 4, 128, 128, 1, 1, 0.1, 0, None]
    assert lib.gdn_recurrent_fwd_gating(*P, *G[:3], None, 1, 1, 0, 1.0, 20.0, *rtail) == -1
    assert lib.gdn_recurrent_fwd_gating(*P, *G, 1, 1, 9, 1.0, 20.0, *rtail) == -2
