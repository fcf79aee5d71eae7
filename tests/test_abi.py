"""C-ABI checks that need no GPU: the library loads, exports every function
include/mtx.h declares, the ctypes table matches the header, and invalid
arguments are rejected on the host before any HIP call."""
import ctypes as C
import re
from pathlib import Path

import pytest

from minitorch_amd import _lib as L

HEADER = Path(__file__).resolve().parents[1] / "include" / "mtx.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mtx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_something():
    names = declared_functions()
    assert "mtx_attn_fwd" in names and "mtx_attn_bwd" in names


def test_every_declared_symbol_is_exported_and_bound():
    lib = L.lib()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in mtx.h but not exported"
        assert name in L.SIGNATURES, f"{name} has no ctypes signature in _lib.py"
    assert set(L.SIGNATURES) == set(declared_functions())


def test_version():
    assert b"gfx950" in L.lib().mtx_version()


def _strides(*s):
    return (C.c_int64 * 4)(*s)


def _fwd(**over):
    args = dict(dtype=L.MTX_F32, B=1, H=1, Tq=8, Tk=8, D=64, q=16, qs=(512, 512, 64, 1),
                k=16, ks=(512, 512, 64, 1), v=16, vs=(512, 512, 64, 1), o=16, os=(512, 512, 64, 1),
                lse=16, scale=0.125, causal=1)
    args.update(over)
    a = args
    # fake (never dereferenced) device addresses: validation fails before any HIP call
    p = lambda x: C.c_void_p(x) if x else None
    return L.lib().mtx_attn_fwd(a["dtype"], a["B"], a["H"], a["Tq"], a["Tk"], a["D"],
                                p(a["q"]), _strides(*a["qs"]), p(a["k"]), _strides(*a["ks"]),
                                p(a["v"]), _strides(*a["vs"]), p(a["o"]), _strides(*a["os"]),
                                p(a["lse"]), a["scale"], a["causal"], None)


@pytest.mark.parametrize("over,code,frag", [
    (dict(dtype=7), L.MTX_ERR_DTYPE, "dtype"),
    (dict(D=48), L.MTX_ERR_SHAPE, "head dim"),
    (dict(Tq=0), L.MTX_ERR_SHAPE, ">= 1"),
    (dict(Tq=9, Tk=8), L.MTX_ERR_SHAPE, "Tq <= Tk"),
    (dict(q=0), L.MTX_ERR_ARG, "null"),
    (dict(lse=0), L.MTX_ERR_ARG, "lse"),
    (dict(ks=(512, 512, 64, 2)), L.MTX_ERR_ARG, "d stride"),
    (dict(vs=(512, 512, 66, 1)), L.MTX_ERR_ARG, "multiple"),
    (dict(o=24), L.MTX_ERR_ARG, "aligned"),
    (dict(scale=-1.0), L.MTX_ERR_ARG, "scale"),
    (dict(ks=(1 << 30, 512, 1 << 24, 1)), L.MTX_ERR_SHAPE, "t stride"),
])
def test_attn_fwd_rejects_bad_arguments(over, code, frag):
    rc = _fwd(**over)
    assert rc == code
    assert frag in L.lib().mtx_last_error().decode()


def test_attn_bwd_rejects_small_workspace():
    s = _strides(512, 512, 64, 1)
    p = C.c_void_p(16)
    rc = L.lib().mtx_attn_bwd(L.MTX_F32, 1, 1, 8, 8, 64, p, s, p, s, p, s, p, s, p, s, p,
                              p, s, p, s, p, s, p, 4, 0.125, 1, 0, None)
    assert rc == L.MTX_ERR_ARG
    assert "workspace" in L.lib().mtx_last_error().decode()


def test_attn_bwd_phase_mask_checked():
    s = _strides(512, 512, 64, 1)
    p = C.c_void_p(16)
    rc = L.lib().mtx_attn_bwd_phase(8, L.MTX_F32, 1, 1, 8, 8, 64, p, s, p, s, p, s, p, s, p, s, p,
                                    p, s, p, s, p, s, p, 1 << 20, 0.125, 1, 0, None)
    assert rc == L.MTX_ERR_ARG


def test_workspace_query():
    assert L.lib().mtx_attn_bwd_workspace_bytes(2, 3, 5) == 2 * 3 * 5 * 4
    assert L.lib().mtx_attn_bwd_workspace_bytes(0, 3, 5) == 0


def test_python_wrapper_raises_value_error():
    s = _strides(512, 512, 64, 1)
    p = C.c_void_p(16)
    with pytest.raises(ValueError, match="phase"):
        L.call("mtx_attn_bwd_phase", 0, L.MTX_F32, 1, 1, 8, 8, 64, p, s, p, s, p, s, p, s, p, s, p,
               p, s, p, s, p, s, p, 1 << 20, 0.125, 1, 0, None)


def _dec(**over):
    args = dict(dtype=L.MTX_F32, B=2, H=3, Lk=40, D=64, q=16, qs=(192, 64, 0, 1), k=16,
                ks=(7680, 64, 192, 1), v=16, vs=(7680, 64, 192, 1), o=16, os=(192, 64, 0, 1))
    args.update(over)
    a = args
    p = lambda x: C.c_void_p(x) if x else None
    return L.lib().mtx_attn_decode(a["dtype"], a["B"], a["H"], a["Lk"], a["D"],
                                   p(a["q"]), _strides(*a["qs"]), p(a["k"]), _strides(*a["ks"]),
                                   p(a["v"]), _strides(*a["vs"]), p(a["o"]), _strides(*a["os"]),
                                   None, None, 0.125, None)


@pytest.mark.parametrize("over,code,frag", [
    (dict(dtype=5), L.MTX_ERR_DTYPE, "dtype"),
    (dict(Lk=8193), L.MTX_ERR_SHAPE, "8192"),
    (dict(Lk=-1), L.MTX_ERR_SHAPE, "cached keys"),
    (dict(D=24), L.MTX_ERR_SHAPE, "head dim"),
    (dict(B=0), L.MTX_ERR_SHAPE, "B,H"),
    (dict(k=0), L.MTX_ERR_ARG, "null"),
    (dict(vs=(7680, 64, 192, 2)), L.MTX_ERR_ARG, "d stride"),
    (dict(ks=(7680, 64, 190, 1)), L.MTX_ERR_ARG, "multiple"),
    (dict(o=8), L.MTX_ERR_ARG, "aligned"),
])
def test_attn_decode_rejects_bad_arguments(over, code, frag):
    rc = _dec(**over)
    assert rc == code
    assert frag in L.lib().mtx_last_error().decode()


def test_argmax_rejects_bad_arguments():
    p = C.c_void_p(16)
    assert L.lib().mtx_argmax_f32(4, 65, p, 64, p, 1, None, 0, None) == L.MTX_ERR_ARG
    assert "ld" in L.lib().mtx_last_error().decode()
    assert L.lib().mtx_argmax_f32(0, 65, p, 65, p, 1, None, 0, None) == L.MTX_ERR_SHAPE
    assert L.lib().mtx_argmax_f32(4, 65, None, 65, p, 1, None, 0, None) == L.MTX_ERR_ARG


def _step(**over):
    a = dict(M=64, N=1152, K=384, a=16, lda=384, b=16, ldb=1152, c=16, ldc=384, act=0, nc=384,
             kc=16, vc=16, sb=256 * 384, st=384, T=256, lengths=16)
    a.update(over)
    p = lambda x: C.c_void_p(x) if x else None
    return L.lib().mtx_gemm_step_f32(a["M"], a["N"], a["K"], p(a["a"]), a["lda"], p(a["b"]), a["ldb"], 0.0,
                                     p(a["c"]), a["ldc"], None, a["act"], a["nc"], p(a["kc"]), p(a["vc"]),
                                     a["sb"], a["st"], a["T"], p(a["lengths"]), None)


@pytest.mark.parametrize("over,code,frag", [
    (dict(M=65), L.MTX_ERR_SHAPE, "M <= 64"),
    (dict(K=513, lda=513), L.MTX_ERR_SHAPE, "K <= 512"),
    (dict(M=0), L.MTX_ERR_SHAPE, ">= 1"),
    (dict(act=2), L.MTX_ERR_ARG, "act"),
    (dict(nc=1153), L.MTX_ERR_ARG, "ncols_c"),
    (dict(nc=385, ldc=385), L.MTX_ERR_ARG, "evenly"),
    (dict(kc=0), L.MTX_ERR_ARG, "null cache"),
    (dict(lengths=0), L.MTX_ERR_ARG, "null cache"),
    (dict(st=100), L.MTX_ERR_ARG, "cache strides"),
    (dict(lda=100), L.MTX_ERR_ARG, "row strides"),
    (dict(a=0), L.MTX_ERR_ARG, "null operand"),
])
def test_gemm_step_rejects_bad_arguments(over, code, frag):
    """Every rejection returns before any launch (no GPU needed)."""
    rc = _step(**over)
    assert rc == code
    assert frag in L.lib().mtx_last_error().decode()


def test_captured_step_needs_an_eager_warmup():
    """A recording cannot contain the first call's host -> device uploads."""
    from minitorch_amd.graphs import CapturedStep

    with pytest.raises(ValueError, match="warm-up"):
        CapturedStep(lambda: None, warmup=0)


def _decode_model(n_layer=2, C=384, n_head=6, F=1536, V=65, Tmax=64, B=4, null=None):
    """An mtx_decode_model of fake (never dereferenced) device addresses."""
    layers = (L.DecodeLayer * n_layer)()
    for y in layers:
        for name, _ in L.DecodeLayer._fields_[:14]:
            setattr(y, name, 0x100000)
        y.ln1_eps = y.ln2_eps = 1e-5
    if null is not None:
        setattr(layers[0], null, None)
    m = L.DecodeModel(n_layer, B, C, n_head, F, V, Tmax)
    m.tok_emb = m.pos_emb = m.lnf_gamma = m.lnf_beta = m.w_head = m.b_head = 0x100000
    m.n_tok, m.n_pos, m.lnf_eps = V, Tmax, 1e-5
    m.layers = layers
    return m, layers


@pytest.mark.parametrize("over,code,frag", [
    (dict(C=320, n_head=5), L.MTX_ERR_SHAPE, "C = 64 n_head"),
    (dict(C=384, n_head=4), L.MTX_ERR_SHAPE, "head size 64"),
    (dict(F=1024), L.MTX_ERR_SHAPE, "F = 4C"),
    (dict(V=257), L.MTX_ERR_SHAPE, "V <="),
    (dict(Tmax=1025), L.MTX_ERR_SHAPE, "Tmax"),
    (dict(n_layer=17), L.MTX_ERR_SHAPE, "n_layer"),
    (dict(null="w_fc2"), L.MTX_ERR_ARG, "null pointer in layer 0"),
    (dict(ws=None), L.MTX_ERR_ARG, "workspace"),
    (dict(steps=0), L.MTX_ERR_ARG, "steps"),
])
def test_decode_step_rejects_bad_arguments(over, code, frag):
    """mtx_decode_step_f32 validates the model, the buffers and the workspace
    before any HIP call (no GPU needed)."""
    lib = L.lib()
    ws = over.pop("ws", 0x10000)  # a fake address: every case fails validation before any HIP call
    over_steps = over.pop("steps", 1)
    m, keep = _decode_model(**over)
    need = lib.mtx_decode_step_workspace_bytes(m.B, 384, 6, 1536)
    assert need > 0
    rc = lib.mtx_decode_step_f32(C.addressof(m), over_steps, 0x1000, 0x1000, None, 0, 0, 0x1000, 0x1000, ws,
                                 need, 0, None)
    assert rc == code
    assert frag in lib.mtx_last_error().decode()


def test_decode_step_null_arguments():
    lib = L.lib()
    assert lib.mtx_decode_step_f32(None, 1, 0x1000, 0x1000, None, 0, 0, 0x1000, 0x1000, 0x10000, 1 << 30, 0,
                                   None) == L.MTX_ERR_ARG
    m, keep = _decode_model()
    assert lib.mtx_decode_step_f32(C.addressof(m), 1, None, 0x1000, None, 0, 0, 0x1000, 0x1000, 0x10000,
                                   1 << 30, 0, None) == L.MTX_ERR_ARG
    assert lib.mtx_decode_step_status(None, None) == L.MTX_ERR_ARG
    assert lib.mtx_decode_step_reset(None, None) == L.MTX_ERR_ARG
    assert lib.mtx_decode_step_workspace_bytes(0, 384, 6, 1536) == 0
