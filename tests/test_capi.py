"""The C-ABI library loads and exports every entry point include/tritiercache_amd.h declares.
No compute calls: this runs without a GPU."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tritiercache_amd.h")
LIB = os.path.join(ROOT, "tritiercache_amd", "libtritiercache_amd.so")


def declared_symbols():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"^TT_API\s+[\w\s\*]*?\b(tt_\w+)\s*\(", src, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("tt_fused_attention_decode", "tt_quantize_k_block", "tt_quantize_v_block", "tt_dequantize_k",
              "tt_dequantize_v", "tt_engine_create", "tt_engine_step", "tt_engine_prefill", "tt_engine_buffer"):
        assert s in syms


@pytest.mark.skipif(not os.path.exists(LIB), reason="native library not built")
def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT\s+(tt_\w+)", out))
    missing = [s for s in declared_symbols() if s not in exported]
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(LIB), reason="native library not built")
def test_python_binding_signatures_cover_header():
    from tritiercache_amd import _lib

    assert set(declared_symbols()) == set(_lib.EXPORTED_SYMBOLS)
    lib = _lib.load()
    for s in declared_symbols():
        assert hasattr(lib, s)
    assert lib.tt_version().decode().startswith("tritiercache_amd")


@pytest.mark.skipif(not os.path.exists(LIB), reason="native library not built")
def test_reference_module_surface():
    """The symbols the reference CLI requires of tri_tier._C (src/tri_tier/cli.py:153-160)."""
    from tritiercache_amd import _C

    for s in ("TriTierCacheEngine", "fused_attention_decode", "quantize_k_block", "quantize_v_block", "dequantize_k",
              "dequantize_v"):
        assert hasattr(_C, s)


@pytest.mark.skipif(not os.path.exists(LIB), reason="native library not built")
def test_errors_without_gpu_are_python_exceptions():
    import torch

    from tritiercache_amd import _C

    if torch.cuda.is_available():
        pytest.skip("checks the no-GPU error path")
    with pytest.raises(RuntimeError):
        _C.TriTierCacheEngine(4, 4, 64, 128)
    with pytest.raises(ValueError):
        _C.fused_attention_decode(0, None, None, -1, None, None, None, None, None, None, None, 0, 4, 4, 64, 0)


@pytest.mark.skipif(not os.path.exists(LIB), reason="native library not built")
def test_decode_seq_layout_matches_header(tmp_path):
    """The ctypes mirror of tt_decode_seq has the C struct's size and field offsets (gcc on the header)."""
    import ctypes as C
    import shutil

    from tritiercache_amd import _lib

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    names = [f[0] for f in _lib.DecodeSeq._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "tritiercache_amd.h"\nint main(void) {\n'
                   '  printf("%zu\\n", sizeof(tt_decode_seq));\n'
                   + "".join(f'  printf("%zu\\n", offsetof(tt_decode_seq, {n}));\n' for n in names) + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [C.sizeof(_lib.DecodeSeq)] + [getattr(_lib.DecodeSeq, n).offset for n in names]
    assert got == want


@pytest.mark.skipif(not os.path.exists(LIB), reason="native library not built")
def test_batched_workspace_rejects_bad_shapes():
    """Host-side validation of the batched entry point (no kernel runs)."""
    from tritiercache_amd import _lib

    L = _lib.load()
    seqs = (_lib.DecodeSeq * 2)()
    for s in seqs:
        s.Q, s.attn_output, s.dense_count, s.num_blocks = 0x1000, 0x2000, 0, 0
    assert L.tt_batched_decode_workspace_bytes(seqs, 2, 7, 2, 128, 16) == 0   # GQA ratio not integral
    assert _lib.last_error()
    assert L.tt_batched_decode_workspace_bytes(seqs, -1, 8, 2, 128, 16) == 0
    seqs[1].num_blocks = 3  # PBS pointers missing
    assert L.tt_batched_decode_workspace_bytes(seqs, 2, 8, 2, 128, 16) == 0
    seqs[1].num_blocks = 0
    assert L.tt_batched_decode_workspace_bytes(seqs, 2, 8, 2, 128, 16) > 0


@pytest.mark.skipif(not os.path.exists(LIB), reason="native library not built")
def test_deferred_finalize_validates_before_launching():
    """Host-side validation of tt_attention_finalize_deferred: every rejected call returns before any
    kernel runs (the pointers are placeholders, never dereferenced)."""
    from tritiercache_amd import _lib

    L = _lib.load()
    Hq, Hkv, D, kgs, nd, nb = 32, 8, 128, 16, 300, 120
    need = int(L.tt_fused_attention_workspace_bytes(nd, nb, Hq, Hkv, D, kgs, 1))
    assert need > 0
    q, out, mw = 0x10000, 0x20000, 0x30000
    ws, prev = 0x1000000, 0x1000000 + 2 * need

    def call(**kw):
        a = dict(Q=q, nd=nd, nb=nb, Hq=Hq, Hkv=Hkv, D=D, out=out, kgs=kgs, fp16=0, ws=ws, ws_bytes=need,
                 pnd=nd, pnb=nb, pmw=mw, pws=prev, pws_bytes=need)
        a.update(kw)
        return L.tt_attention_finalize_deferred(a["Q"], a["nd"], a["nb"], a["Hq"], a["Hkv"], a["D"], a["out"],
                                                a["kgs"], a["fp16"], a["ws"], a["ws_bytes"], a["pnd"], a["pnb"],
                                                a["pmw"], a["pws"], a["pws_bytes"], None)

    assert call(out=None) == 1 and "attn_output" in _lib.last_error()
    assert call(pmw=None) == 1 and "prev_mean_attn_weights" in _lib.last_error()
    assert call(pws=ws + need // 2) == 1 and "overlap" in _lib.last_error()
    assert call(pws_bytes=need // 2) == 1 and "smaller" in _lib.last_error()
    assert call(pnb=nb + 500, pws_bytes=need) == 1  # the earlier call's plan needs a larger workspace
    assert call(Hkv=7) == 1  # query heads not a multiple of the KV heads
    assert call(Q=None) == 1


def test_logits_larger_than_4gib_are_rejected():
    """The kernels store the logits of the mean weights through buffer resources (a 32-bit byte range):
    calls whose logits would pass 4 GiB fail on the host, for one sequence, a batch and an engine."""
    import ctypes as C
    from tritiercache_amd import _lib

    L = _lib.load()
    Hq, Hkv, D, kgs = 64, 8, 128, 16
    nd_big = (1 << 32) // (4 * Hq) + 16  # one row of Hq logits past 4 GiB
    p = 0x10000
    rc = L.tt_attention_partials(p, p, p, nd_big, p, p, p, p, p, p, p, 0, Hq, Hkv, D, kgs, 0, 1, p, 1 << 62, None)
    assert rc == 1 and "4 GiB" in _lib.last_error()
    # without mean weights there are no logits, and the same call passes validation (its workspace is too small)
    rc = L.tt_attention_partials(p, p, p, nd_big, p, p, p, p, p, p, p, 0, Hq, Hkv, D, kgs, 0, 0, p, 256, None)
    assert rc == 1 and "4 GiB" not in _lib.last_error()

    seqs = (_lib.DecodeSeq * 2)()
    for i, (nd, mw) in enumerate([(300, p), (nd_big, p)]):
        s = seqs[i]
        s.Q, s.dense_K, s.dense_V = p, p, p
        s.PBS_K_Packed = s.PBS_K_Scales = s.PBS_K_Zeroes = s.PBS_V_Packed = s.PBS_V_Scales = s.PBS_V_Zeroes = p
        s.PBS_token_ids, s.attn_output, s.mean_attn_weights = p, p, mw
        s.dense_count, s.num_blocks = nd, 4
    assert L.tt_batched_decode_workspace_bytes(seqs, 2, Hq, Hkv, D, kgs) == 0
    assert "4 GiB" in _lib.last_error()
    seqs[1].mean_attn_weights = None
    assert L.tt_batched_decode_workspace_bytes(seqs, 2, Hq, Hkv, D, kgs) > 0

    eng = C.c_void_p()
    rc = L.tt_engine_create(C.byref(eng), Hq, Hkv, D, nd_big, 4, 256, 0.05, 0.999, 32, kgs, b"fp32", None)
    assert rc == 1 and "4 GiB" in _lib.last_error() and not eng.value


def test_workspace_size_query_validates_like_the_entry_points():
    """tt_fused_attention_workspace_bytes returns 0 and sets the error for arguments the attention entry
    points reject, including token counts past int and logits past 4 GiB, and a size otherwise."""
    from tritiercache_amd import _lib

    L = _lib.load()
    q = L.tt_fused_attention_workspace_bytes
    for args, msg in [((-1, 5, 32, 8, 128, 16, 1), "dense_count"), ((10, -2, 32, 8, 128, 16, 1), "num_blocks"),
                      ((10, 5, 32, 7, 128, 16, 1), "multiple"), ((10, 5, 32, 8, 72, 16, 1), "head_dim"),
                      ((10, 5, 32, 8, 272, 16, 1), "head_dim"),
                      ((10, 5, 32, 8, 128, 24, 1), "k_group_size"),
                      ((1 << 30, 1 << 26, 64, 8, 128, 32, 1), "2^31"),
                      ((1 << 28, 0, 64, 8, 128, 16, 1), "4 GiB")]:
        assert q(*args) == 0 and msg in _lib.last_error(), (args, _lib.last_error())
    assert q(1 << 28, 0, 64, 8, 128, 16, 0) > 0  # no mean weights: no logits
    assert q(300, 120, 32, 8, 128, 16, 1) > 0 and _lib.last_error() == ""
    assert q(300, 120, 32, 8, 96, 16, 1) > 0 and _lib.last_error() == ""  # any multiple of 16 up to 256
    # the entry points reject the same token count
    p = 0x10000
    rc = L.tt_attention_partials(p, p, p, 1 << 30, p, p, p, p, p, p, p, 1 << 26, 64, 8, 128, 32, 0, 0, p, 1 << 40, None)
    assert rc == 1 and "2^31" in _lib.last_error()
