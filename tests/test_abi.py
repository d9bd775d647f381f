"""The C ABI without a GPU: libprism_kv.so loads, exports every function include/prism_kv.h declares,
the binding's constants match the header, and argument checks fail before anything is launched.

No call here reaches the HIP runtime: each one is rejected by the host-side validation that runs
first (or, for pkv_decode_workspace_bytes, takes a path that only does arithmetic).
"""
import ctypes
import re

import pytest

from prism_amd import _lib

HEADER = _lib.HEADER_PATH.read_text()


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built (python -m prism_amd.build)")
    return _lib.load()


def test_library_exports_every_header_function(lib):
    names = _lib.header_symbols()
    assert len(names) >= 8, names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in prism_kv.h but not exported"
        assert name in _lib._SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib._SIGNATURES) == set(names)


def test_header_constants_match_binding(lib):
    defines = dict(re.findall(r"^#define (PKV_\w+) \(?(-?\d+)\)?", HEADER, re.M))
    for name in ["PKV_OK", "PKV_EINVAL", "PKV_EHIP", "PKV_ENOSPC", "PKV_STATUS_BAD_PAGE", "PKV_STATUS_BAD_POSITION",
                 "PKV_STATUS_SHARED_PREFIX", "PKV_STATUS_PARTIAL_RANGE", "PKV_STATUS_MERGE_TIMEOUT", "PKV_DECODE_TWO_PASS",
                 "PKV_DECODE_FUSED_MERGE", "PKV_DECODE_HEADS", "PKV_DECODE_RESET_COUNTERS"]:
        assert int(defines[name]) == getattr(_lib, name), name
    assert int(defines["PKV_ABI_VERSION"]) == _lib.ABI_VERSION == lib.pkv_abi_version()
    assert lib.pkv_last_error() == b""


A16 = 1 << 20  # a 16-byte-aligned stand-in address: never dereferenced, every call below is rejected first


def _decode(lib, **over):
    a = dict(q=A16, q_sb=28 * 128, q_ss=28 * 128, q_sh=128, k=A16, k_sb=512, k_ss=512, k_sh=128,
             v=A16, v_sb=512, v_ss=512, v_sh=128, kc=A16, vc=A16, page_stride=256 * 512, bt=A16, bt_stride=4,
             sl=A16, out=A16, o_sb=28 * 128, o_ss=28 * 128, o_sh=128, ws=A16, ws_bytes=0, batch=2, s_q=1,
             n_heads=28, n_kv=4, head_dim=128, page_size=256, num_pages=10, max_blocks=4, causal=1, scale=0.088,
             split=0, flags=0)
    a.update(over)
    return lib.pkv_decode_attn(a["q"], a["q_sb"], a["q_ss"], a["q_sh"], a["k"], a["k_sb"], a["k_ss"], a["k_sh"],
                               a["v"], a["v_sb"], a["v_ss"], a["v_sh"], a["kc"], a["vc"], a["page_stride"],
                               a["bt"], a["bt_stride"], a["sl"], a["out"], a["o_sb"], a["o_ss"], a["o_sh"],
                               a["ws"], a["ws_bytes"], a["batch"], a["s_q"], a["n_heads"], a["n_kv"],
                               a["head_dim"], a["page_size"], a["num_pages"], a["max_blocks"], a["causal"],
                               a["scale"], a["split"], a["flags"], None, None)


@pytest.mark.parametrize("over,msg", [
    (dict(head_dim=96, q_sh=96, k_sh=96, v_sh=96, o_sh=96), "head_dim"),
    (dict(page_size=48), "page_size"),
    (dict(page_size=8), "page_size"),
    (dict(bt_stride=3), "bt_stride"),
    (dict(kc=A16 + 8), "aligned"),
    (dict(q=A16 + 2), "aligned"),
    (dict(q_ss=28 * 128 + 4), "multiples of 8"),
    (dict(n_heads=30), "multiple of n_kv"),
    (dict(s_q=10), "> 64"),
    (dict(split=48), "multiple of 32"),
    (dict(flags=3), "bad flags"),
    (dict(flags=1 << 30), "bad flags"),
    (dict(k=0), "both be given"),
    (dict(scale=0.0), "softmax_scale"),
    (dict(max_blocks=(1 << 19) + 1, bt_stride=(1 << 19) + 1), "2^27 keys"),
    (dict(bt=0), "null"),
    (dict(num_pages=0), "bad sizes"),
    (dict(page_stride=100), "page stride"),
])
def test_decode_argument_errors(lib, over, msg):
    rc = _decode(lib, **over)
    assert rc == _lib.PKV_EINVAL
    err = lib.pkv_last_error().decode()
    assert "pkv_decode_attn" in err and msg in err, err


def test_decode_workspace_too_small_is_enospc(lib):
    # the per-head kernel (split_tokens > 0) with two splits needs a workspace
    rc = _decode(lib, split=256, ws=A16, ws_bytes=64)
    assert rc == _lib.PKV_ENOSPC
    assert "workspace" in lib.pkv_last_error().decode()


def test_workspace_bytes_arithmetic(lib):
    # head_dim 64 with an odd n_kv never takes the balanced kernel (nor does a fixed split_tokens),
    # so this is pure arithmetic: counters (64 KiB) + batch * n_kv * splits * R * (head_dim + 2)
    # floats
    f = lib.pkv_decode_workspace_bytes
    assert f(0, 1, 14, 1, 64, 256, 4, 0) == 0
    assert f(2, 1, 14, 1, 64, 256, 2, 0) == 0          # 512 keys fit the default 512-key split
    B, s_q, nh, nkv, hd, P, mb, st = 3, 1, 14, 2, 64, 256, 8, 256
    R = s_q * nh // nkv
    splits = -(-(mb * P) // st)
    assert f(B, s_q, nh, nkv, hd, P, mb, st) == 65536 + B * nkv * splits * R * (hd + 2) * 4
    # the balanced kernel's bound (one workgroup per CU; 256 without a GPU): counters + 2 slots per
    # workgroup of 4 heads x R rows x (256 B of fp16 + a 4-byte log-sum-exp), for every geometry
    # it serves, or the per-head kernel's need where that is larger
    for nh, nkv, hd in [(28, 4, 128), (7, 1, 128), (14, 2, 128), (14, 2, 64), (28, 4, 64), (40, 8, 128)]:
        R = nh // nkv
        per_head = 65536 + 2 * nkv * 4 * R * (hd + 2) * 4  # batch 2, 4 splits of 512 keys
        assert f(2, 1, nh, nkv, hd, 256, 8, 0) == max(65536 + 2 * 256 * 4 * R * 260, per_head)


def test_copy_and_gather_argument_errors(lib):
    rc = lib.pkv_copy_pages(A16, A16, 2, A16, A16, None, 3, 1000, 1 << 18, 1024, 256, 10, 10, None, None)
    assert rc == _lib.PKV_EINVAL and "pkv_copy_pages" in lib.pkv_last_error().decode()
    rc = lib.pkv_copy_pages(A16, A16, 2, A16, None, None, 3, 1 << 18, 1 << 18, 1024, 256, 10, 10, None, None)
    assert rc == _lib.PKV_EINVAL and "dst_ids" in lib.pkv_last_error().decode()
    rc = lib.pkv_gather_pages(A16, A16, 2, A16, 3, 0, 1 << 18, 1 << 18, 1000, 10, 10, None, None)
    assert rc == _lib.PKV_EINVAL and "pkv_gather_pages" in lib.pkv_last_error().decode()


def test_append_argument_errors(lib):
    rc = lib.pkv_append(A16, 512, 512, 128, A16, 512, 512, 128, A16, A16, 256 * 512, A16, 4, A16,
                        2, 1, 4, 80, 256, 10, 4, None, None)
    assert rc == _lib.PKV_EINVAL and "head_dim" in lib.pkv_last_error().decode()
    rc = lib.pkv_append(A16 + 4, 512, 512, 128, A16, 512, 512, 128, A16, A16, 256 * 512, A16, 4, A16,
                        2, 1, 4, 128, 256, 10, 4, None, None)
    assert rc == _lib.PKV_EINVAL and "aligned" in lib.pkv_last_error().decode()


def test_errors_are_thread_local_and_cleared(lib):
    assert _decode(lib, head_dim=96) == _lib.PKV_EINVAL
    assert lib.pkv_last_error() != b""
    seen = {}

    def other():
        seen["err"] = lib.pkv_last_error()

    import threading

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["err"] == b""
    # a later call that fails differently replaces the message
    assert _decode(lib, page_size=48) == _lib.PKV_EINVAL
    assert "page_size" in lib.pkv_last_error().decode()


def test_ctypes_types_are_c_abi_only():
    # the ABI carries plain pointers, integers and floats only (no torch types)
    allowed = {ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float, ctypes.c_char_p}
    for name, (res, args) in _lib._SIGNATURES.items():
        assert res in allowed, name
        assert all(a in allowed for a in args), name


def _decode_noalloc(lib, **over):
    a = dict(q=A16, q_sb=28 * 128, q_ss=28 * 128, q_sh=128, k=A16, k_sb=512, k_ss=512, k_sh=128,
             v=A16, v_sb=512, v_ss=512, v_sh=128, kc=A16, vc=A16, page_stride=256 * 512, bt=A16, bt_stride=4,
             sl=A16, out=A16, o_sb=28 * 128, o_ss=28 * 128, o_sh=128, batch=2, s_q=1, n_heads=28, n_kv=4,
             head_dim=128, page_size=256, num_pages=10, max_blocks=4, causal=1, scale=0.088, split=0, flags=0)
    a.update(over)
    return lib.pkv_decode_attn_noalloc(a["q"], a["q_sb"], a["q_ss"], a["q_sh"], a["k"], a["k_sb"], a["k_ss"],
                                       a["k_sh"], a["v"], a["v_sb"], a["v_ss"], a["v_sh"], a["kc"], a["vc"],
                                       a["page_stride"], a["bt"], a["bt_stride"], a["sl"], a["out"], a["o_sb"],
                                       a["o_ss"], a["o_sh"], a["batch"], a["s_q"], a["n_heads"], a["n_kv"],
                                       a["head_dim"], a["page_size"], a["num_pages"], a["max_blocks"], a["causal"],
                                       a["scale"], a["split"], a["flags"], None, None)


def test_noalloc_rejects_before_any_device_work(lib):
    # argument errors: the same checks as pkv_decode_attn, named for the variant
    for over, msg in [(dict(head_dim=96, q_sh=96, k_sh=96, v_sh=96, o_sh=96), "head_dim"), (dict(s_q=10), "> 64"),
                      (dict(flags=3), "bad flags"), (dict(split=48), "multiple of 32")]:
        assert _decode_noalloc(lib, **over) == _lib.PKV_EINVAL
        err = lib.pkv_last_error().decode()
        assert "pkv_decode_attn_noalloc" in err and msg in err, err
    # a call whose split-K partials exceed the 48 MiB static scratch: PKV_ENOSPC, with the size
    over = dict(batch=256, n_kv=8, n_heads=64, k_sh=128, q_sh=128, q_sb=64 * 128, q_ss=64 * 128, o_sb=64 * 128,
                o_ss=64 * 128, k_sb=1024, k_ss=1024, v_sb=1024, v_ss=1024, page_stride=256 * 1024, max_blocks=64,
                bt_stride=64, split=256)
    need = lib.pkv_decode_workspace_bytes(256, 1, 64, 8, 128, 256, 64, 256)
    assert need > 48 << 20
    assert _decode_noalloc(lib, **over) == _lib.PKV_ENOSPC
    err = lib.pkv_last_error().decode()
    assert "static scratch" in err and str(need) in err, err


def test_stamps_library_is_the_same_abi_plus_its_readers():
    """bench.py --workload tile-stamps swaps libprism_kv_stamps.so in for libprism_kv.so: it must
    export every header function with the same ABI version, and its three stamp readers."""
    from prism_amd.build import STAMPS_LIB_PATH

    if not STAMPS_LIB_PATH.exists():
        pytest.fail(f"{STAMPS_LIB_PATH} is not built (python -m prism_amd.build)")
    slib = ctypes.CDLL(str(STAMPS_LIB_PATH))
    for name in _lib.header_symbols():
        assert hasattr(slib, name), f"{name} missing from the stamps build"
    slib.pkv_abi_version.restype = ctypes.c_int32
    assert slib.pkv_abi_version() == _lib.ABI_VERSION
    for name in ("pkv_tile_stamps", "pkv_tile_stamps_clear", "pkv_tile_stamp_words"):
        assert hasattr(slib, name), name
    slib.pkv_tile_stamp_words.restype = ctypes.c_int
    words = slib.pkv_tile_stamp_words()
    assert words == 1024 * 32 + 4 * 4096
    # too small a destination is rejected before any HIP call
    slib.pkv_tile_stamps.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    assert slib.pkv_tile_stamps(ctypes.c_void_p(A16), 8, None) == _lib.PKV_EINVAL
