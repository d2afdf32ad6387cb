"""The C ABI of libaicas_decode.so, on the CPU: the library loads, exports every entry point that
include/aicas_decode.h declares, plans launches, and rejects bad arguments with the documented codes.

No call here reaches a kernel launch: argument checks run before anything touches a device, so the fake
device addresses below are never dereferenced.
"""

import ctypes
import os
import re
import subprocess

import pytest

from aicas_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "aicas_decode.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(aicas_\w+)\s*\(", text, flags=re.M)


def test_header_declarations_are_exported():
    lib = _lib.lib()
    declared = _declared_functions()
    assert sorted(declared) == sorted(_lib.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version_matches_header():
    m = re.search(r"#define AICAS_ABI_VERSION (\d+)", open(HEADER).read())
    assert int(m.group(1)) == _lib.ABI_VERSION == _lib.lib().aicas_abi_version()


def test_constants_match_header():
    text = open(HEADER).read()
    for name, value in [("AICAS_DTYPE_BF16", _lib.DTYPE_BF16), ("AICAS_DTYPE_FP16", _lib.DTYPE_FP16),
                        ("AICAS_DTYPE_FP8_E4M3", _lib.DTYPE_FP8_E4M3), ("AICAS_ERR_INVALID", _lib.ERR_INVALID),
                        ("AICAS_ERR_UNSUPPORTED", _lib.ERR_UNSUPPORTED), ("AICAS_ERR_WORKSPACE", _lib.ERR_WORKSPACE),
                        ("AICAS_ERR_LAUNCH", _lib.ERR_LAUNCH), ("AICAS_STATUS_LEN_CLAMPED", _lib.STATUS_LEN_CLAMPED),
                        ("AICAS_STATUS_BLOCK_OUT_OF_RANGE", _lib.STATUS_BLOCK_OUT_OF_RANGE),
                        ("AICAS_STATUS_APPEND_OVERFLOW", _lib.STATUS_APPEND_OVERFLOW),
                        ("AICAS_STATUS_OUT_OF_BLOCKS", _lib.STATUS_OUT_OF_BLOCKS),
                        ("AICAS_STATUS_NONFINITE_ROW", _lib.STATUS_NONFINITE_ROW)]:
        assert re.search(rf"#define {name} {value}\b", text), name


@pytest.mark.parametrize("ctype, struct", [("aicas_kv_cache_t", _lib.KVCacheDesc),
                                           ("aicas_qk_prologue_t", _lib.QKPrologueDesc),
                                           ("aicas_block_pool_t", _lib.BlockPoolDesc)])
def test_descriptor_layouts_match_header(tmp_path, ctype, struct):
    """The ctypes mirrors of the ABI's structs have the C compiler's layout (sizeof and every offsetof)."""
    fields = [f[0] for f in struct._fields_]
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "aicas_decode.h"\nint main(void) {\n'
        + f'  printf("%zu\\n", sizeof({ctype}));\n'
        + "".join(f'  printf("%zu\\n", offsetof({ctype}, {f}));\n' for f in fields)
        + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    subprocess.run(["gcc", "-D__HIP_PLATFORM_AMD__", "-I", os.path.dirname(HEADER), "-I", os.path.join(rocm, "include"),
                    str(src), "-o", str(exe)], check=True)
    values = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert values[0] == ctypes.sizeof(struct)
    for f, off in zip(fields, values[1:]):
        assert getattr(struct, f).offset == off, f


def _plan(kv_dtype, B, Hq, Hkv, D, L, page=0, hint=0):
    tps, ns, wb = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_size_t()
    rc = _lib.lib().aicas_decode_plan(kv_dtype, B, Hq, Hkv, D, L, page, hint, ctypes.byref(tps), ctypes.byref(ns),
                                      ctypes.byref(wb))
    return rc, tps.value, ns.value, wb.value


@pytest.mark.parametrize("B, Hkv, L", [(8, 8, 2113), (1, 8, 32832), (64, 8, 4097), (32, 8, 8193), (1, 2, 1)])
def test_plan_covers_every_token(B, Hkv, L):
    """A sequence of L tokens takes min(num_splits, ceil(L / tokens_per_split)) splits: at least one, never more
    than planned; the split size is a whole number of workgroup loads; the workspace holds every split's
    partial."""
    for kv in (_lib.DTYPE_BF16, _lib.DTYPE_FP8_E4M3):
        rc, tps, ns, wb = _plan(kv, B, 2 * Hkv, Hkv, 128, L)
        assert rc == _lib.OK
        assert ns >= 1 and 1 <= min(ns, -(-L // tps)) <= ns
        rows = 16 if kv == _lib.DTYPE_BF16 else 32  # tokens one workgroup load covers at D=128
        assert tps % rows == 0
        parts = B * 2 * Hkv * ns
        assert wb >= parts * (128 + 2) * 4 + B * Hkv * 4 + B * 4


@pytest.mark.skipif(__import__("torch").cuda.is_available(), reason="pins the plan for 256 compute units")
def test_plan_split_counts():
    """The planner's measured choices for 256 compute units: with few (batch, kv head) pairs about 7/8 of a
    workgroup per CU and never more than one (64 splits per pair for at most 4 pairs), with many pairs 7/4, and at
    least one super-chunk per wave."""
    bf, f8 = _lib.DTYPE_BF16, _lib.DTYPE_FP8_E4M3
    assert _plan(bf, 8, 16, 8, 128, 2176)[2] == 4      # B=8 L=2048 + 128 steps: 256 workgroups
    assert _plan(bf, 1, 16, 8, 128, 32832)[2] == 28    # B=1 L=32768 + 64 steps: 224 workgroups
    assert _plan(bf, 1, 16, 8, 128, 1025)[1:3] == (128, 9)  # B=1 L=1024: 128 tokens = 4 waves x 32
    # at most 4 pairs: 64 splits per pair once the sequence is long enough (1, 2 and 4 kv heads)
    assert _plan(bf, 1, 2, 1, 128, 32768)[2] == _plan(bf, 1, 4, 2, 128, 16384)[2] == 64
    assert _plan(bf, 1, 8, 4, 128, 8192)[2] == 64 and _plan(bf, 1, 8, 4, 128, 4096)[2] == 32
    assert _plan(f8, 32, 16, 8, 128, 8193, 16)[2] == 2  # 256 pairs: 7/4 per CU
    assert _plan(bf, 64, 16, 8, 128, 4097)[2] == 1     # 512 pairs
    # few pairs: the split size is the minimum (two chunks per wave) and the count does not follow a loose bound
    assert _plan(bf, 8, 16, 8, 128, 2049)[1:3] == _plan(bf, 8, 16, 8, 128, 65536)[1:3] == (128, 4)
    assert _plan(bf, 1, 16, 8, 128, 32769)[1:3] == _plan(bf, 1, 16, 8, 128, 1 << 20)[1:3] == (128, 28)
    # many pairs: in proportion to the bound, so that the longest sequences split
    assert _plan(bf, 64, 16, 8, 128, 8192)[2] == 1 and _plan(f8, 32, 16, 8, 128, 4096, 16)[2] == 2
    for B in range(1, 25):
        for L in (300, 2049, 9000):
            rc, tps, ns, _ = _plan(bf, B, 16, 8, 128, L)
            assert rc == _lib.OK and tps >= 128
            if B * 8 * 4 <= 3 * 256:
                assert B * 8 * ns <= 256, (B, L, ns)


def test_plan_honours_hint_and_rejects_bad_shapes():
    rc, tps, ns, _ = _plan(_lib.DTYPE_BF16, 8, 16, 8, 128, 2113, hint=300)
    assert rc == _lib.OK and tps == 304 and ns == 7
    assert _plan(_lib.DTYPE_BF16, 8, 16, 8, 96, 100)[0] == _lib.ERR_UNSUPPORTED
    assert _plan(7, 8, 16, 8, 128, 100)[0] == _lib.ERR_UNSUPPORTED
    assert _plan(_lib.DTYPE_BF16, 0, 16, 8, 128, 100)[0] == _lib.ERR_INVALID
    # at most 65536 (batch row, kv head) pairs per launch: the workspace's counter region holds that many
    assert _plan(_lib.DTYPE_BF16, 8192, 16, 8, 128, 32)[0] == _lib.OK
    assert _plan(_lib.DTYPE_BF16, 8193, 16, 8, 128, 32)[0] == _lib.ERR_UNSUPPORTED


FAKE = 0x7F0000000000  # a 16-byte-aligned address that is never dereferenced

# The argument-error tests below pass fake device addresses; they must never be able to reach a launch on a
# real GPU, so they only run where there is none (the CPU suite).
no_gpu_only = pytest.mark.skipif(
    __import__("torch").cuda.is_available(), reason="fake device addresses are only passed where no GPU exists"
)


def _desc(dtype=_lib.DTYPE_BF16, cap=64, D=128, H=8):
    d = _lib.KVCacheDesc()
    d.k = FAKE
    d.v = FAKE + (1 << 24)
    d.stride_h = cap * D
    d.stride_blk = H * cap * D
    d.stride_t = D
    d.page_size = cap
    d.kv_dtype = dtype
    d.num_blocks = 1
    return d


def _decode(desc, **over):
    args = dict(q_dtype=_lib.DTYPE_BF16, q=FAKE, qsb=16 * 128, qsh=128, out=FAKE + 4096, osb=16 * 128, osh=128,
                seq_lens=None, uniform=10, min_len=0, max_len=10, B=1, Hq=16, Hkv=8, D=128, scale=0.1, tps=0,
                ws=FAKE + (1 << 26), wsb=1 << 20, status=None, stream=None)
    args.update(over)
    return _lib.lib().aicas_decode_attention(
        ctypes.byref(desc) if desc is not None else None, args["q_dtype"], args["q"], args["qsb"], args["qsh"],
        args["out"], args["osb"], args["osh"], args["seq_lens"], args["uniform"], args["min_len"], args["max_len"],
        args["B"], args["Hq"], args["Hkv"], args["D"], args["scale"], args["tps"], args["ws"], args["wsb"],
        args["status"], args["stream"])


def _last_error():
    return _lib.lib().aicas_last_error().decode()


@no_gpu_only
@pytest.mark.parametrize("over, code, msg", [
    (dict(q_dtype=5), _lib.ERR_UNSUPPORTED, "q must be bf16 or fp16"),
    (dict(q=None), _lib.ERR_INVALID, "non-NULL"),
    (dict(q=FAKE + 2), _lib.ERR_INVALID, "16-byte aligned"),
    (dict(Hq=12), _lib.ERR_INVALID, "multiple of num_kv_heads"),
    (dict(D=96), _lib.ERR_UNSUPPORTED, "head_dim"),
    (dict(ws=None), _lib.ERR_WORKSPACE, "workspace is NULL"),
    (dict(wsb=64), _lib.ERR_WORKSPACE, "needed"),
    (dict(q_dtype=_lib.DTYPE_FP16), _lib.ERR_UNSUPPORTED, "dtype of q"),
    (dict(Hq=8 * 3), _lib.ERR_UNSUPPORTED, "group size"),
])
def test_decode_argument_errors(over, code, msg):
    assert _decode(_desc(), **over) == code
    assert msg in _last_error()


@no_gpu_only
def test_decode_cache_descriptor_errors():
    assert _decode(None) == _lib.ERR_INVALID
    d = _desc()
    d.stride_t = 100  # 200 bytes: not a multiple of 16
    assert _decode(d) == _lib.ERR_INVALID and "multiples of 16 bytes" in _last_error()
    d = _desc(dtype=_lib.DTYPE_FP8_E4M3)
    assert _decode(d) == _lib.ERR_INVALID and "k_scale" in _last_error()
    d = _desc()
    d.block_table = FAKE
    d.page_size = 24
    d.block_table_stride = 4
    assert _decode(d) == _lib.ERR_INVALID and "power-of-two" in _last_error()


@no_gpu_only
def test_append_argument_errors():
    lib = _lib.lib()
    d = _desc()

    def call(**over):
        a = dict(src=_lib.DTYPE_BF16, k=FAKE, v=FAKE, pos=FAKE, B=1, H=8, D=128, n=1, ks=8 * 128, kh=128, kt=128)
        a.update(over)
        return lib.aicas_kv_append(ctypes.byref(d), a["src"], a["k"], a["ks"], a["kh"], a["kt"], a["v"], a["ks"],
                                   a["kh"], a["kt"], a["pos"], None, None, a["B"], a["H"], a["D"], a["n"], None)

    assert call(n=0) == _lib.ERR_INVALID
    assert call(pos=None) == _lib.ERR_INVALID
    assert call(src=_lib.DTYPE_FP8_E4M3) == _lib.ERR_UNSUPPORTED
    assert call(src=_lib.DTYPE_FP16) == _lib.ERR_UNSUPPORTED and "dtype of the new rows" in _last_error()
    assert call(kh=100) == _lib.ERR_INVALID
    assert call(D=48) == _lib.ERR_UNSUPPORTED
    # the kernel's row strides are 32-bit, its row indexes 31-bit
    assert call(kh=1 << 32) == _lib.ERR_UNSUPPORTED and "[0, 2^32)" in _last_error()
    assert call(n=1 << 27, H=8) == _lib.ERR_UNSUPPORTED and "too many rows" in _last_error()


@no_gpu_only
def test_fused_entry_argument_errors():
    lib = _lib.lib()
    d = _desc()
    rc = lib.aicas_decode_attention_append(
        ctypes.byref(d), _lib.DTYPE_BF16, FAKE, 16 * 128, 128, FAKE, 8 * 128, 128, FAKE, 8 * 128, 128,
        FAKE + 4096, 16 * 128, 128, None, None, 0, 10, 1, 16, 8, 128, 0.1, 0, FAKE, 1 << 20, None, None)
    assert rc == _lib.ERR_INVALID and "positions" in _last_error()
    rc = lib.aicas_decode_attention_append(
        ctypes.byref(d), _lib.DTYPE_BF16, FAKE, 16 * 128, 128, None, 8 * 128, 128, FAKE, 8 * 128, 128,
        FAKE + 4096, 16 * 128, 128, FAKE, None, 0, 10, 1, 16, 8, 128, 0.1, 0, FAKE, 1 << 20, None, None)
    assert rc == _lib.ERR_INVALID and "k_new" in _last_error()
    # seq_lens_out may be positions itself, never a shifted view of it
    rc = lib.aicas_decode_attention_append(
        ctypes.byref(d), _lib.DTYPE_BF16, FAKE, 16 * 128, 128, FAKE, 8 * 128, 128, FAKE, 8 * 128, 128,
        FAKE + 4096, 16 * 128, 128, FAKE + 256, FAKE + 260, 0, 10, 2, 16, 8, 128, 0.1, 0, FAKE, 1 << 20, None, None)
    assert rc == _lib.ERR_INVALID and "overlap" in _last_error()


@no_gpu_only
def test_fused_qk_entry_argument_errors():
    lib = _lib.lib()
    d = _desc()

    def call(pro):
        return lib.aicas_decode_attention_append_qk(
            ctypes.byref(d), pro, _lib.DTYPE_BF16, FAKE, 16 * 128, 128, FAKE, 8 * 128, 128, FAKE, 8 * 128, 128,
            FAKE + 4096, 16 * 128, 128, FAKE, None, 0, 10, 1, 16, 8, 128, 0.1, 0, FAKE + (1 << 26), 1 << 20, None,
            None)

    assert call(None) == _lib.ERR_INVALID and "prologue" in _last_error()
    pro = _lib.QKPrologueDesc()
    pro.cos = FAKE
    assert call(ctypes.byref(pro)) == _lib.ERR_INVALID and "cos and sin" in _last_error()
    pro = _lib.QKPrologueDesc()
    pro.q_norm_weight = FAKE + 2
    assert call(ctypes.byref(pro)) == _lib.ERR_INVALID and "aligned" in _last_error()
    pro = _lib.QKPrologueDesc()
    pro.q_norm_weight = FAKE
    pro.eps = -1.0
    assert call(ctypes.byref(pro)) == _lib.ERR_INVALID and "eps" in _last_error()


def test_block_pool_argument_errors():
    """Every rejected argument returns before anything reaches the GPU."""
    lib = _lib.lib()
    pool = _lib.BlockPoolDesc(FAKE, FAKE + 4096, 16)

    def alloc(p=pool, table=FAKE + 8192, stride=4, width=4, pos=FAKE + 12288, n_new=1, batch=2, page=16):
        return lib.aicas_block_alloc(ctypes.byref(p) if p is not None else None, table, stride, width, pos, n_new,
                                     batch, page, None, None)

    assert alloc(p=None) == _lib.ERR_INVALID and "pool" in _last_error()
    assert alloc(p=_lib.BlockPoolDesc(FAKE, FAKE + 4096, 0)) == _lib.ERR_INVALID and "num_blocks" in _last_error()
    assert alloc(table=None) == _lib.ERR_INVALID and "block_table" in _last_error()
    assert alloc(width=0) == _lib.ERR_INVALID and "width" in _last_error()
    assert alloc(stride=2) == _lib.ERR_INVALID and "stride" in _last_error()
    assert alloc(pos=None) == _lib.ERR_INVALID and "positions" in _last_error()
    assert alloc(n_new=0) == _lib.ERR_INVALID and "n_new" in _last_error()
    assert alloc(page=12) == _lib.ERR_INVALID and "power of two" in _last_error()
    assert alloc(batch=-1) == _lib.ERR_INVALID and "batch" in _last_error()
    assert alloc(batch=0) == 0  # nothing to do: no launch
    assert lib.aicas_block_free(ctypes.byref(pool), FAKE + 8192, 4, 4, None, None, 2, None, None) == _lib.ERR_INVALID
    assert "release" in _last_error()
    assert lib.aicas_block_pool_init(None, None) == _lib.ERR_INVALID
