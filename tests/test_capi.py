"""The C-ABI library on the CPU: it loads, exports every symbol include/ccinfer_attn.h
declares, and rejects invalid arguments before touching a device (the reference's
DeviceBackend / launcher validation, src/backend/backend.h:172-223,
src/kernel/attention/decode_attn.cu:488,568, prefill_attn.cu:257-259)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from ccinfer_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ccinfer_attn.h"
INVALID = 6
FAKE = 0x1000  # never dereferenced: every call below fails validation first


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ccinfer_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 7
    for n in names:
        assert hasattr(lib, n), n
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                        text=True, check=True).stdout
    exported = set(re.findall(r"\bT (ccinfer_\w+)", nm))
    assert set(names) <= exported
    assert set(names) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"


def test_version_and_messages(lib):
    assert lib.ccinfer_version().decode().count(".") == 2
    assert lib.ccinfer_error_message(0) == b"ok"
    assert lib.ccinfer_error_message(INVALID) == b"invalid argument"


def test_write_kv_cache_validation(lib):
    f = lib.ccinfer_write_kv_cache
    assert f(None, FAKE, FAKE, FAKE, FAKE, 4, 2, 4, 64, None) == INVALID
    assert f(FAKE, FAKE, FAKE, FAKE, None, 4, 2, 4, 64, None) == INVALID
    for bad in [(0, 2, 4, 64), (4, 0, 4, 64), (4, 2, 0, 64), (4, 2, 4, 0), (-1, 2, 4, 64)]:
        assert f(FAKE, FAKE, FAKE, FAKE, FAKE, *bad, None) == INVALID


def _decode(lib, **kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, bt=FAKE, ctx=FAKE, out=FAKE, b=2, mbpr=4, hq=8, hkv=2,
             d=128, bs=16, ws=None, wsb=0)
    a.update(kw)
    return lib.ccinfer_decode_attention(a["q"], a["k"], a["v"], a["bt"], a["ctx"], a["out"],
                                        a["b"], a["mbpr"], a["hq"], a["hkv"], a["d"], a["bs"],
                                        a["ws"], a["wsb"], None)


def test_decode_validation(lib):
    for ptr in ["q", "k", "v", "bt", "ctx", "out"]:
        assert _decode(lib, **{ptr: None}) == INVALID, ptr
    for field in ["b", "mbpr", "hq", "hkv", "d", "bs"]:
        assert _decode(lib, **{field: 0}) == INVALID, field
    assert _decode(lib, hq=7) == INVALID              # Hq % Hkv != 0
    assert _decode(lib, bs=32) == INVALID             # decode_attn.cu:488
    assert _decode(lib, d=100) == INVALID             # decode_attn.cu:568
    # split-KV needs a workspace for this shape; a missing one is rejected, not allocated
    need = lib.ccinfer_decode_workspace_size(64, 256, 16, 8, 128, 16)
    assert need > 0
    assert _decode(lib, b=64, mbpr=256, hq=16, hkv=8, ws=None, wsb=0) == INVALID
    # an aligned call needs the size without the q / output row copies, a call with a
    # 2-byte-aligned q or output the whole size
    aligned = need - _row_copies(64, 16, 128)
    assert _decode(lib, b=64, mbpr=256, hq=16, hkv=8, ws=FAKE, wsb=aligned - 1) == INVALID
    for ptr in ("q", "out"):
        assert _decode(lib, b=64, mbpr=256, hq=16, hkv=8, ws=FAKE, wsb=need - 1,
                       **{ptr: FAKE + 2}) == INVALID, ptr


def test_decode_write_kv_validation(lib):
    f = lib.ccinfer_decode_attention_write_kv
    ok = [FAKE] * 8 + [2, 4, 16, 8, 128, 16, 1024, None, 0, None]
    for i in range(8):                     # q, k_new, v_new, caches, table, ctx, output
        a = list(ok)
        a[i] = None
        assert f(*a) == INVALID, i
    a = list(ok)
    a[14] = 0                              # max_slots
    assert f(*a) == INVALID
    a = list(ok)
    a[12] = 100                            # not a decode head dim
    assert f(*a) == INVALID
    a = list(ok)
    a[8], a[9] = 64, 256                   # needs a workspace: a missing one is rejected
    assert f(*a) == INVALID


def _row_copies(b, hq, d):
    """Two 256-byte-aligned copies of the q rows, at the end of every MFMA-path workspace
    (used only by calls whose q or output view is 2-byte aligned)."""
    return 2 * ((b * hq * d * 2 + 255) // 256 * 256)


def test_decode_workspace_size(lib):
    def f(b, mbpr, hq, hkv, d, bs):
        n = lib.ccinfer_decode_workspace_size(b, mbpr, hq, hkv, d, bs)
        return n - _row_copies(b, hq, d) if n else n
    assert f(0, 4, 8, 2, 128, 16) == 0            # invalid shape -> 0
    assert f(1, 1, 8, 2, 128, 16) == 0            # one 16-token block: single split, no scratch
    assert f(7, 2, 8, 2, 128, 16) == 0            # 32 tokens: one chunk per request
    # partials ((D + 2) floats per partial row), then a 16-byte merge descriptor per (B, Hq)
    n = f(32, 2048, 32, 8, 128, 16) - 32 * 32 * 16
    assert n > 0 and n % (32 * 130 * 4) == 0      # Hq * partial slots * (D + 2) floats
    assert n <= 32 * 32 * 2048 * 130 * 4          # never more than one slot per 32 tokens
    big = f(300, 2048, 32, 8, 128, 16) - 300 * 32 * 16  # flat plan with its index kernel
    assert big >= 300 * 32 * 130 * 4                    # at least one partial slot per row
    # head_dim 80 runs the MFMA kernels at 128 with zero padding: partial rows of 128 floats
    assert f(32, 2048, 32, 8, 80, 16) == f(32, 2048, 32, 8, 128, 16)
    assert f(32, 2048, 32, 8, 72, 16) == 0        # not a decode head dim: invalid shape


def test_prefill_workspace_size_for_other_block_sizes(lib):
    """Blocks of 16·k tokens run the MFMA prefill through a 16-token table built in the
    workspace: the size is that of the 16-token shape plus the table. Other block sizes run
    the any-layout tile kernel: the planner's tile list only, the same for every block size
    and table length."""
    f = lib.ccinfer_prefill_workspace_size
    base = f(4, 512, 64, 16, 8, 128, 16)
    assert base > 0
    for k in (2, 4, 16):
        n = f(4, 512, 64 // k, 16, 8, 128, 16 * k)
        table = (4 * 64 * 4 + 255) // 256 * 256
        assert n == base + table, k
    any8 = f(4, 512, 64, 16, 8, 128, 8)
    assert 0 < any8 < base
    assert f(4, 512, 64, 16, 8, 128, 24) == any8
    assert f(4, 512, 64, 16, 8, 100, 16) > 0       # head dim 100: any-layout kernel
    assert f(4, 512, 5000, 16, 8, 128, 8) == any8  # any table length


def _prefill(lib, **kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, bt=FAKE, qsl=FAKE, ctx=FAKE, out=FAKE, b=2, t=64, mbpr=8,
             hq=16, hkv=8, d=128, bs=16, ws=None, wsb=0)
    a.update(kw)
    return lib.ccinfer_prefill_attention(a["q"], a["k"], a["v"], a["bt"], a["qsl"], a["ctx"],
                                         a["out"], a["b"], a["t"], a["mbpr"], a["hq"], a["hkv"],
                                         a["d"], a["bs"], a["ws"], a["wsb"], None)


def test_prefill_validation(lib):
    for ptr in ["q", "k", "v", "bt", "qsl", "ctx", "out"]:
        assert _prefill(lib, **{ptr: None}) == INVALID, ptr
    for field in ["b", "t", "mbpr", "hq", "hkv", "d", "bs"]:
        assert _prefill(lib, **{field: 0}) == INVALID, field
    assert _prefill(lib, hq=12) == INVALID             # 12 % 8 != 0
    assert _prefill(lib, d=264) == INVALID             # prefill_attn.cu:257-259
    need = lib.ccinfer_prefill_workspace_size(2, 64, 8, 16, 8, 128, 16)
    assert need > 0
    assert _prefill(lib) == INVALID                     # workspace missing
    assert _prefill(lib, ws=FAKE, wsb=need - _row_copies(64, 16, 128) - 1) == INVALID
    assert _prefill(lib, ws=FAKE, wsb=need - 1, q=FAKE + 2) == INVALID


def test_alignment_limits_and_overlap_validation(lib):
    """fp8 calls (MFMA path only) reject q / output / cache / scale pointers that are not
    16-byte aligned; bf16 calls take them on other routes (GPU tests). Large batches
    and long tables stay on the MFMA prefill (nonzero workspace); the fp8 prefill keeps its
    4096-block table limit; a side stream without its events is rejected."""
    UNSUPPORTED = 26
    d8 = lib.ccinfer_decode_attention_fp8
    args = [FAKE] * 8 + [2, 4, 8, 2, 128, 16, None, 0, None]
    for i in (0, 1, 2, 3, 4, 7):          # q, k, v, k_scale, v_scale, output
        a = list(args)
        a[i] = FAKE + (2 if i < 3 or i == 7 else 4)
        assert d8(*a) == INVALID, i
    p8 = lib.ccinfer_prefill_attention_fp8
    pargs = [FAKE] * 9 + [2, 64, 8, 16, 8, 128, 16, FAKE, 1 << 30, None]
    for i in (0, 1, 8):                   # q, k_cache, output
        a = list(pargs)
        a[i] = FAKE + 8
        assert p8(*a) == INVALID, i
    a = list(pargs)
    a[11] = 5000                          # more than 4096 blocks per row
    assert p8(*a) == UNSUPPORTED
    assert lib.ccinfer_prefill_workspace_size(6000, 6000, 8, 16, 8, 128, 16) > 0
    assert lib.ccinfer_prefill_workspace_size(2, 64, 8192, 16, 8, 128, 16) > 0
    # head dim 256 past 4096 table blocks: the any-layout tile kernel (ids read from the
    # table row in global memory)
    assert lib.ccinfer_prefill_workspace_size(2, 64, 8192, 16, 8, 256, 16) > 0
    ov = lib.ccinfer_prefill_attention_overlap
    base = [FAKE] * 7 + [2, 64, 8, 16, 8, 128, 16, FAKE, 1 << 30, None]
    assert ov(*base, FAKE, None, FAKE) == INVALID
    assert ov(*base, FAKE, FAKE, None) == INVALID
    ov8 = lib.ccinfer_prefill_attention_fp8_overlap
    assert ov8(*pargs, FAKE, None, None) == INVALID


def test_error_code_values_match_reference_enum():
    """The C ABI returns the reference's ErrorCode numbering (src/base/error_code.h:8-45)."""
    text = (ROOT / "ccinfer_amd" / "csrc" / "dropin" / "base" / "error_code.h").read_text()
    body = text[text.index("enum class ErrorCode"):]
    body = body[body.index("{") + 1:body.index("};")]
    names = [n.strip().split("=")[0].strip() for n in body.split(",") if n.strip()]
    hdr = HEADER.read_text()
    for code, ename in [("CCINFER_ERR_DEVICE_OUT_OF_MEMORY", "CudaOutOfMemory"),
                        ("CCINFER_ERR_LAUNCH_FAILED", "CudaLaunchFailed"),
                        ("CCINFER_ERR_DEVICE_INVALID_VALUE", "CudaInvalidValue"),
                        ("CCINFER_ERR_DEVICE_RUNTIME", "CudaRuntimeError"),
                        ("CCINFER_ERR_INVALID_ARGUMENT", "InvalidArgument"),
                        ("CCINFER_ERR_UNSUPPORTED", "Unsupported"),
                        ("CCINFER_ERR_INTERNAL", "InternalError")]:
        val = int(re.search(rf"{code}\s*=\s*(\d+)", hdr).group(1))
        assert names.index(ename) == val, (code, ename)
    assert ctypes.sizeof(ctypes.c_size_t) == 8


def _prologue(lib, **kw):
    a = dict(qkv=FAKE, qw=FAKE, kw=FAKE, pos=FAKE, rc=FAKE, sm=FAKE, qo=FAKE, kc=FAKE, vc=FAKE,
             t=4, nq=8, nkv=2, d=128, mp=64, slots=64, eps=1e-6)
    a.update(kw)
    return lib.ccinfer_qkv_prologue(a["qkv"], a["qw"], a["kw"], a["pos"], a["rc"], a["sm"],
                                    a["qo"], a["kc"], a["vc"], a["t"], a["nq"], a["nkv"],
                                    a["d"], a["mp"], a["slots"], a["eps"], None)


def test_qkv_prologue_validation(lib):
    for ptr in ["qkv", "pos", "rc", "sm", "qo", "kc", "vc"]:
        assert _prologue(lib, **{ptr: None}) == INVALID, ptr
    for field in ["t", "nq", "nkv", "d", "mp", "slots"]:
        assert _prologue(lib, **{field: 0}) == INVALID, field
    assert _prologue(lib, d=127) == INVALID           # RoPE pairs need an even head_dim
    assert _prologue(lib, d=1026) == INVALID
    assert _prologue(lib, eps=0.0) == INVALID         # backend.h:84
    assert _prologue(lib, eps=float("nan")) == INVALID


def _meta(lib, **kw):
    a = dict(kvw=FAKE, nt=FAKE, fl=FAKE, bst=FAKE, blk=FAKE, b=4, t=8, nb=6, mbpr=4, bs=16,
             ncb=64, pos=FAKE, sm=FAKE, bt=FAKE, qsl=FAKE, ctx=FAKE, li=FAKE, st=FAKE)
    a.update(kw)
    return lib.ccinfer_build_batch_metadata(
        a["kvw"], a["nt"], a["fl"], a["bst"], a["blk"], a["b"], a["t"], a["nb"], a["mbpr"],
        a["bs"], a["ncb"], a["pos"], a["sm"], a["bt"], a["qsl"], a["ctx"], a["li"], a["st"], None)


def test_build_batch_metadata_validation(lib):
    for ptr in ["kvw", "nt", "fl", "bst", "blk", "pos", "sm", "bt", "qsl", "ctx", "li", "st"]:
        assert _meta(lib, **{ptr: None}) == INVALID, ptr
    for field in ["b", "t", "mbpr", "bs", "ncb"]:
        assert _meta(lib, **{field: 0}) == INVALID, field
    assert _meta(lib, nb=-1) == INVALID
    assert _meta(lib, b=1 << 16, mbpr=1 << 16) == INVALID      # table entries overflow int
    assert _meta(lib, ncb=1 << 28, bs=16) == INVALID           # cache slots overflow int


def test_fp8_validation(lib):
    w = lib.ccinfer_write_kv_cache_fp8
    ok = [FAKE] * 7 + [4, 2, 128, 64, None]
    for i in range(7):
        a = list(ok)
        a[i] = None
        assert w(*a) == INVALID, i
    for i, bad in ((7, 0), (8, 0), (9, 0), (9, 127), (9, 514), (10, 0)):
        a = list(ok)
        a[i] = bad
        assert w(*a) == INVALID, (i, bad)
    dec = lib.ccinfer_decode_attention_fp8
    okd = [FAKE] * 8 + [2, 4, 8, 2, 128, 16, None, 0, None]
    for i in range(8):
        a = list(okd)
        a[i] = None
        assert dec(*a) == INVALID, i
    a = list(okd)
    a[12] = 96  # valid decode head dim, but fp8 has the MFMA path only
    assert dec(*a) == 26  # CCINFER_ERR_UNSUPPORTED
    a = list(okd)
    a[13] = 32
    assert dec(*a) == INVALID


def test_prefill_fp8_validation(lib):
    pf = lib.ccinfer_prefill_attention_fp8
    need = lib.ccinfer_prefill_workspace_size(2, 64, 8, 16, 8, 128, 16)
    ok = [FAKE] * 9 + [2, 64, 8, 16, 8, 128, 16, FAKE, need, None]
    assert need > 0
    for i in range(9):
        a = list(ok)
        a[i] = None
        assert pf(*a) == INVALID, i
    for i in range(9, 16):
        a = list(ok)
        a[i] = 0
        assert pf(*a) == INVALID, i
    a = list(ok)
    a[14] = 96                   # a valid bf16 prefill head dim; fp8 is MFMA-only (64 / 128)
    assert pf(*a) == 26          # CCINFER_ERR_UNSUPPORTED
    a = list(ok)
    a[17] = need - _row_copies(64, 16, 128) - 1   # fp8 views are aligned: no row copies
    assert pf(*a) == INVALID
    a = list(ok)
    a[16] = None
    assert pf(*a) == INVALID
