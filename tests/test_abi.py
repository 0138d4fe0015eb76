"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares with the expected arity, and the host-side argument checks
return the documented status codes before anything is enqueued (the analogue
of the `bail!` checks in crane-core/src/fused_ops/cuda_impl.rs:61-72)."""
import ctypes
import os
import re

import pytest

from crane_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def _declared():
    decls = {}
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
        for m in re.finditer(r"\b(?:int|void|size_t|int64_t|uint64_t|const char\s*\*)\s+(crane_\w+)\s*"
                             r"\(([^)]*)\)\s*;", text):
            args = [a for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
            decls[m.group(1)] = len(args)
    return decls


def test_header_declares_the_path():
    d = _declared()
    assert {"crane_hip_strerror", "crane_hip_version", "crane_hip_qknorm_rope_append",
            "crane_hip_attn_decode_workspace", "crane_hip_attn_decode", "crane_hip_attn_prefill"} <= set(d)
    assert {"crane_kv_grown_capacity", "crane_kv_create", "crane_kv_destroy", "crane_kv_reserve",
            "crane_kv_update", "crane_kv_append_qkv", "crane_kv_decode", "crane_kv_prefill", "crane_kv_views",
            "crane_kv_set_lengths", "crane_kv_bytes", "crane_kv_stack", "crane_kv_extract"} <= set(d)
    assert set(d) == set(_lib.SIGNATURES), set(d) ^ set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name, nargs in _declared().items():
        assert hasattr(L, name), name
        assert len(_lib.SIGNATURES[name][0]) == nargs, name


def test_one_hip_runtime_per_process():
    """Loading the library before torch must not leave two HIP runtimes in the
    process (torch carries its own libamdhip64; the library's runpath names
    the /opt/rocm one): the loader brings torch's in first.  Run in a fresh
    interpreter, where nothing has imported torch yet."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from crane_amd import _lib\n"
            "_lib.lib()\n"
            "import torch\n"
            "maps = open('/proc/self/maps').read().split('\\n')\n"
            "print(len({l.split()[-1] for l in maps if 'libamdhip64' in l}))\n") % ROOT
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().splitlines()[-1] == "1", out.stdout


def test_strerror_and_version():
    assert _lib.version().startswith("crane_hip 2 gfx950")
    for code in range(0, 9):
        assert _lib.strerror(code)
    assert "capacity" in _lib.strerror(_lib.E_CAPACITY)
    assert _lib.strerror(99) == "unknown crane_hip status"


def _decode(**kw):
    a = dict(q=16, k=16, v=16, cap=4096, kv_len=16, max_kv=4096, B=1, Hq=32, Hkv=8, D=128, scale=0.088,
             score=_lib.SCORE_GROUPED, ws=16, ws_bytes=1 << 30, out=16, dtype=1, stream=None)
    a.update(kw)
    return _lib.lib().crane_hip_attn_decode(a["q"], a["k"], a["v"], a["cap"], a["kv_len"], a["max_kv"], a["B"],
                                            a["Hq"], a["Hkv"], a["D"], a["scale"], a["score"], a["ws"],
                                            a["ws_bytes"], a["out"], a["dtype"], a["stream"])


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=2), _lib.E_DTYPE),
    (dict(D=64), _lib.E_HEAD_DIM),
    (dict(Hq=30), _lib.E_GQA),
    (dict(max_kv=5000), _lib.E_CAPACITY),
    (dict(max_kv=0), _lib.E_INVALID),
    (dict(scale=0.0), _lib.E_INVALID),
    (dict(score=2), _lib.E_INVALID),
    (dict(score=-1), _lib.E_INVALID),
    (dict(q=None), _lib.E_INVALID),
    (dict(q=8), _lib.E_ALIGN),
    (dict(ws_bytes=100), _lib.E_WORKSPACE),
    (dict(ws=None), _lib.E_WORKSPACE),
    (dict(B=0), _lib.OK),                 # empty batch: nothing to do
])
def test_decode_argument_checks(kw, code):
    assert _decode(**kw) == code


@pytest.mark.parametrize("B,Hq,Hkv,max_kv", [(32, 32, 8, 4097), (8, 64, 8, 32769), (1, 16, 8, 1025)])
def test_decode_workspace_size(B, Hq, Hkv, max_kv):
    """[B, Hq, splits, D] partial rows in the call's dtype (bf16 rows for bf16
    calls, f32 for f32), then [B, Hq, splits, 2] f32 (max, sum) pairs; one split
    per 256 keys."""
    L = _lib.lib()
    ns = (max_kv + 255) // 256
    up = lambda x: (x + 255) // 256 * 256
    assert L.crane_hip_attn_decode_workspace(B, Hq, Hkv, 128, max_kv, 1) == up(B * Hq * ns * 128 * 2) + up(B * Hq * ns * 8)
    assert L.crane_hip_attn_decode_workspace(B, Hq, Hkv, 128, max_kv, 0) == up(B * Hq * ns * 128 * 4) + up(B * Hq * ns * 8)
    assert L.crane_hip_attn_decode_workspace(32, 32, 8, 64, 4096, 1) == 0
    assert L.crane_hip_attn_decode_workspace(0, 32, 8, 128, 4096, 1) == 0
    assert L.crane_hip_attn_decode_workspace(32, 32, 8, 128, 4096, 7) == 0


def _prefill(**kw):
    a = dict(q=16, k=16, v=16, cap=4096, start=16, max_start=0, B=1, S=2048, Hq=16, Hkv=8, D=128, scale=0.088,
             causal=1, out=16, dtype=1, stream=None)
    a.update(kw)
    return _lib.lib().crane_hip_attn_prefill(a["q"], a["k"], a["v"], a["cap"], a["start"], a["max_start"], a["B"],
                                             a["S"], a["Hq"], a["Hkv"], a["D"], a["scale"], a["causal"], a["out"],
                                             a["dtype"], a["stream"])


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=5), _lib.E_DTYPE),
    (dict(D=256), _lib.E_HEAD_DIM),
    (dict(Hkv=3), _lib.E_GQA),
    (dict(max_start=2049), _lib.E_CAPACITY),
    (dict(S=4097), _lib.E_CAPACITY),
    (dict(max_start=-1), _lib.E_INVALID),
    (dict(out=None), _lib.E_INVALID),
    (dict(k=24), _lib.E_ALIGN),
    (dict(S=0), _lib.OK),
])
def test_prefill_argument_checks(kw, code):
    assert _prefill(**kw) == code


def _append(**kw):
    a = dict(qkv=16, stride=4096, qw=None, kw=None, eps=1e-6, order=0, cos=16, sin=16, cs_stride=64,
             rows=40960, pos=16, q_out=16, kc=16, vc=16, cap=4096, clen=16, max_rows=4096, B=1, S=2048,
             Hq=16, Hkv=8, D=128, dtype=1, stream=None)
    a.update(kw)
    return _lib.lib().crane_hip_qknorm_rope_append(
        a["qkv"], a["stride"], a["qw"], a["kw"], a["eps"], a["order"], a["cos"], a["sin"], a["cs_stride"],
        a["rows"], a["pos"], a["q_out"], a["kc"], a["vc"], a["cap"], a["clen"], a["max_rows"], a["B"], a["S"],
        a["Hq"], a["Hkv"], a["D"], a["dtype"], a["stream"])


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=3), _lib.E_DTYPE),
    (dict(D=96), _lib.E_HEAD_DIM),
    (dict(Hkv=5), _lib.E_GQA),
    (dict(order=3), _lib.E_INVALID),
    (dict(max_rows=4097), _lib.E_CAPACITY),
    (dict(S=5000, max_rows=4096), _lib.E_CAPACITY),
    (dict(stride=4000), _lib.E_INVALID),
    (dict(stride=4098), _lib.E_ALIGN),
    (dict(cs_stride=32), _lib.E_INVALID),
    (dict(rows=0), _lib.E_INVALID),
    (dict(cos=None), _lib.E_INVALID),
    (dict(qw=20), _lib.E_ALIGN),
    (dict(eps=-1.0), _lib.E_INVALID),
    (dict(S=0), _lib.OK),
])
def test_append_argument_checks(kw, code):
    assert _append(**kw) == code


def _append_parts(**kw):
    a = dict(parts=16, n=2, bias=None, qw=None, kw=None, eps=1e-6, order=0, cos=16, sin=16, cs_stride=64,
             rows=40960, pos=16, q_out=16, kc=16, vc=16, cap=4096, clen=16, max_rows=4096, B=32, S=1,
             Hq=32, Hkv=8, D=128, dtype=1, stream=None)
    a.update(kw)
    return _lib.lib().crane_hip_qknorm_rope_append_parts(
        a["parts"], a["n"], a["bias"], a["qw"], a["kw"], a["eps"], a["order"], a["cos"], a["sin"], a["cs_stride"],
        a["rows"], a["pos"], a["q_out"], a["kc"], a["vc"], a["cap"], a["clen"], a["max_rows"], a["B"], a["S"],
        a["Hq"], a["Hkv"], a["D"], a["dtype"], a["stream"])


@pytest.mark.parametrize("kw,code", [
    (dict(n=3), _lib.E_INVALID),               # 2 or 4 splits
    (dict(n=1), _lib.E_INVALID),
    (dict(n=3, S=0), _lib.E_INVALID),
    (dict(dtype=3), _lib.E_DTYPE),
    (dict(D=96), _lib.E_HEAD_DIM),
    (dict(Hkv=5), _lib.E_GQA),
    (dict(max_rows=4097), _lib.E_CAPACITY),
    (dict(parts=None), _lib.E_INVALID),
    (dict(parts=20), _lib.E_ALIGN),
    (dict(bias=24), _lib.E_ALIGN),
    (dict(cos=None), _lib.E_INVALID),
    (dict(cs_stride=32), _lib.E_INVALID),
    (dict(S=0), _lib.OK),
    (dict(parts=None, B=0), _lib.OK),
])
def test_append_parts_argument_checks(kw, code):
    assert _append_parts(**kw) == code


def _qnorm(**kw):
    a = dict(q=16, stride=2048, qw=None, eps=1e-6, order=1, cos=16, sin=16, cs_stride=64, rows=40960, pos=16,
             q_out=16, B=1, S=2048, Hq=16, D=128, dtype=1, stream=None)
    a.update(kw)
    return _lib.lib().crane_hip_qnorm_rope(
        a["q"], a["stride"], a["qw"], a["eps"], a["order"], a["cos"], a["sin"], a["cs_stride"], a["rows"], a["pos"],
        a["q_out"], a["B"], a["S"], a["Hq"], a["D"], a["dtype"], a["stream"])


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=2), _lib.E_DTYPE),
    (dict(D=64), _lib.E_HEAD_DIM),
    (dict(Hq=0), _lib.E_INVALID),
    (dict(order=-1), _lib.E_INVALID),
    (dict(stride=2000), _lib.E_INVALID),       # narrower than Hq*D
    (dict(stride=2050), _lib.E_ALIGN),
    (dict(cs_stride=60), _lib.E_INVALID),
    (dict(q_out=None), _lib.E_INVALID),
    (dict(pos=None), _lib.E_INVALID),
    (dict(qw=24), _lib.E_ALIGN),
    (dict(eps=float("nan")), _lib.E_INVALID),
    (dict(B=0), _lib.OK),
    (dict(S=0), _lib.OK),
])
def test_qnorm_rope_argument_checks(kw, code):
    assert _qnorm(**kw) == code


def test_ops_reject_cpu_tensors():
    import torch
    from crane_amd import ops
    q = torch.zeros(1, 8, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 16, 128, dtype=torch.bfloat16)
    with pytest.raises(_lib.CraneHipError, match="GPU only"):
        ops.attention_decode(q, k, k, torch.ones(1, dtype=torch.int32), 16)


def test_kv_stack_and_extract_reject_aliasing():
    """A batch cache cannot be its own source (crane_kv_stack releases dst's
    buffer before copying) or its own extraction target; both are rejected on
    the host before any device call."""
    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.crane_kv_create(1, 8, 128, _lib.BF16, ctypes.byref(h)) == _lib.OK
    try:
        srcs = (ctypes.c_void_p * 1)(h.value)
        assert L.crane_kv_stack(h, srcs, 1, 0, None) == _lib.E_INVALID
        assert L.crane_kv_extract(h, 0, h, None) == _lib.E_INVALID
        assert L.crane_kv_stack(h, None, 1, 0, None) == _lib.E_INVALID
    finally:
        L.crane_kv_destroy(h)
