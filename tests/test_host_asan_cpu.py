"""Host-side AddressSanitizer run of the C ABI (no GPU).

The library is rebuilt with the host code instrumented (the device code is
compiled as usual) and loaded, with the ASan runtime preloaded, in a child
process that does not import torch.  The child drives every entry point's
host validation: argument checks, pointer arrays, workspace-size
arithmetic and the per-thread error string.  Every call fails validation
before any device work (pointers are placeholders that are never
dereferenced), so no GPU is needed.  Any ASan report fails the test.
"""

import os
import shutil
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ASAN_RT = "/opt/rocm/llvm/lib/clang/22/lib/linux/libclang_rt.asan-x86_64.so"

CHILD = textwrap.dedent('''
    import ctypes, importlib.util, sys
    spec = importlib.util.spec_from_file_location("abi", sys.argv[1])
    abi = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(abi)
    L = abi.bind(ctypes.CDLL(sys.argv[2]))
    P = 0x10000   # placeholder address: every call below returns before using it
    EINVAL, EWS = -1, -2

    def err(rc, want, name):
        assert rc == want, (name, rc, want)
        msg = L.swattn_last_error()
        assert msg and name.encode() in msg, (name, msg)

    assert L.swattn_version() > 0
    assert L.swattn_compact_workspace_bytes(100000) > 0
    assert L.swattn_compact_workspace_bytes(-1) == 0
    err(L.swattn_compact(None, 10, P, P, P, 1 << 20, None), EINVAL, "swattn_compact")
    err(L.swattn_compact_logits(P, 7, 10, 0.0, P, P, P, 1 << 20, None), EINVAL,
        "swattn_compact_logits")
    err(L.swattn_check_indices(P, -1, P, 3, 10, P, None), EINVAL, "swattn_check_indices")
    err(L.swattn_check_indices(None, 5, P, 3, 10, P, None), EINVAL, "swattn_check_indices")
    err(L.swattn_build_metadata(P, None, 2, 10, 10, 0, P, P, P, P, P, P, P, None), EINVAL,
        "swattn_build_metadata")
    err(L.swattn_build_metadata(None, None, 2, 10, 10, 4, P, P, P, P, P, P, P, None), EINVAL,
        "swattn_build_metadata")
    assert L.swattn_prefill_workspace_bytes(1, 16384, 8, 128) == 8 * 256 * 16384
    assert L.swattn_prefill_split_workspace_bytes(1, 16384, 16384, 4, 1, 128, 1024, 4028,
                                                  12356) > 256 * 16384
    assert L.swattn_prefill_split_workspace_bytes(1, 16384, 16384, 4, 1, 128, 0, 4028, 12356) == 0
    assert L.swattn_prefill_workspace_bytes(1, 16384, 8, 64) == 0
    fwd = lambda hd, hq, w, ws: L.swattn_prefill_fwd(
        P, P, P, P, 100, P, 100, None, None, None, P, P, 1, 200, 200, hq, 8, hd, w, 0.1, P, ws,
        None)
    err(fwd(64, 32, 64, 1 << 30), EINVAL, "swattn_prefill_fwd")
    err(fwd(128, 33, 64, 1 << 30), EINVAL, "swattn_prefill_fwd")
    err(fwd(128, 32, 0, 1 << 30), EINVAL, "swattn_prefill_fwd")
    err(fwd(128, 32, 64, 16), EWS, "swattn_prefill_fwd")
    err(L.swattn_prefill_fwd(P, P, P, P, 100, P, 100, P, None, None, P, P, 1, 200, 200, 32, 8,
                             128, 64, 0.1, P, 1 << 30, None), EINVAL, "swattn_prefill_fwd")
    wsb = L.swattn_prefill_bwd_workspace_bytes(1, 200, 32, 8, 128, 64, 100, 100)
    assert wsb > 0 and L.swattn_prefill_bwd_workspace_bytes(1, 200, 32, 8, 64, 64, 100, 100) == 0
    assert L.swattn_prefill_bwd_workspace_bytes(1, 200, 32, 8, 128, -1, 100, 100) == 0
    bwd = lambda hd, ws: L.swattn_prefill_bwd(
        P, P, P, P, P, P, P, 100, P, 100, None, None, None, P, P, P, 1, 200, 200, 32, 8, hd, 64,
        0.1, P, ws, None)
    err(bwd(64, wsb), EINVAL, "swattn_prefill_bwd")
    err(bwd(128, wsb - 1), EWS, "swattn_prefill_bwd")
    assert L.swattn_decode_workspace_bytes(0, 100, 32, 8) == 0
    dec = lambda hd, hq: L.swattn_decode_fwd(P, P, P, P, P, P, P, 4, 100, hq, 2, hd, 64, 0.1,
                                             P, 1 << 30, None)
    err(dec(64, 8), EINVAL, "swattn_decode_fwd")
    err(dec(128, 32), EINVAL, "swattn_decode_fwd")     # group 16 > 8
    dna = lambda b, hd, hq: L.swattn_decode_fwd_noalloc(P, P, P, P, P, P, P, b, 100, hq, 2, hd,
                                                        64, 0.1, None)
    err(dna(4, 64, 8), EINVAL, "swattn_decode_fwd_noalloc")
    err(dna(4, 128, 32), EINVAL, "swattn_decode_fwd_noalloc")
    err(dna(65535, 128, 16), EINVAL, "swattn_decode_fwd_noalloc")   # scratch too small
    assert b"scratch" in L.swattn_last_error()
    err(L.swattn_shard_bounds(P, 10, 5, 2, 64, P, P, P, None), EINVAL, "swattn_shard_bounds")
    parts = (ctypes.c_void_p * 2)(P, None)
    lses = (ctypes.c_void_p * 2)(P, P)
    err(L.swattn_merge_partials(parts, lses, 2, P, P, 10, 128, None), EINVAL,
        "swattn_merge_partials")
    err(L.swattn_merge_partials(parts, lses, 17, P, P, 10, 128, None), EINVAL,
        "swattn_merge_partials")
    # bf16 row tensors must be 16-byte aligned (a bf16 view can be 2-aligned)
    M = P + 2
    def unaligned(rc, name):
        err(rc, EINVAL, name)
        assert b"16-byte aligned" in L.swattn_last_error(), L.swattn_last_error()
    unaligned(L.swattn_prefill_fwd(P, M, P, P, 100, P, 100, None, None, None, P, P, 1, 200, 200,
                                   32, 8, 128, 64, 0.1, P, 1 << 30, None), "swattn_prefill_fwd")
    unaligned(L.swattn_prefill_bwd(P, P, P, P, P, M, P, 100, P, 100, None, None, None, P, P, P,
                                   1, 200, 200, 32, 8, 128, 64, 0.1, P, wsb, None),
              "swattn_prefill_bwd")
    unaligned(L.swattn_prefill_bwd(P, P, P, P, P, P, P, 100, P, 100, None, None, None, P, P, M,
                                   1, 200, 200, 32, 8, 128, 64, 0.1, P, wsb, None),
              "swattn_prefill_bwd")
    unaligned(L.swattn_decode_fwd(P, P, M, P, P, P, P, 4, 100, 8, 2, 128, 64, 0.1, P, 1 << 30,
                                  None), "swattn_decode_fwd")
    unaligned(L.swattn_decode_fwd_noalloc(M, P, P, P, P, P, P, 4, 100, 8, 2, 128, 64, 0.1, None),
              "swattn_decode_fwd_noalloc")
    parts = (ctypes.c_void_p * 2)(P, M)
    unaligned(L.swattn_merge_partials(parts, lses, 2, P, P, 10, 128, None),
              "swattn_merge_partials")
    parts = (ctypes.c_void_p * 2)(P, P)
    unaligned(L.swattn_merge_partials(parts, lses, 2, M, P, 10, 128, None),
              "swattn_merge_partials")
    # workspaces must be 256-byte aligned
    W = P + 16
    def ws_unaligned(rc, name):
        err(rc, EINVAL, name)
        assert b"256-byte aligned" in L.swattn_last_error(), L.swattn_last_error()
    ws_unaligned(L.swattn_prefill_fwd(P, P, P, P, 100, P, 100, None, None, None, P, P, 1, 200,
                                      200, 32, 8, 128, 64, 0.1, W, 1 << 30, None),
                 "swattn_prefill_fwd")
    ws_unaligned(L.swattn_prefill_bwd(P, P, P, P, P, P, P, 100, P, 100, None, None, None, P, P,
                                      P, 1, 200, 200, 32, 8, 128, 64, 0.1, W, wsb, None),
                 "swattn_prefill_bwd")
    ws_unaligned(L.swattn_decode_fwd(P, P, P, P, P, P, P, 4, 100, 8, 2, 128, 64, 0.1, W, 1 << 30,
                                     None), "swattn_decode_fwd")
    ws_unaligned(L.swattn_compact(P, 100000, P, P, W, 1 << 20, None), "swattn_compact")
    print("host checks ok")
''')


@pytest.mark.skipif(not (os.path.exists(ASAN_RT) and shutil.which("hipcc") or
                         os.path.exists("/opt/rocm/bin/hipcc")),
                    reason="needs hipcc and the clang ASan runtime")
def test_c_abi_host_paths_under_asan(tmp_path):
    if not os.path.exists(ASAN_RT):
        pytest.skip("clang ASan runtime not found")
    sys.path.insert(0, ROOT)
    from switchattentionkernels_amd import build as B

    lib = B.build(out=str(tmp_path / "libswattn_asan.so"),
                  extra_flags=["-Xarch_host", "-fsanitize=address",
                               "-Xarch_host", "-fno-omit-frame-pointer"])
    script = tmp_path / "child.py"
    script.write_text(CHILD)
    env = dict(os.environ, LD_PRELOAD=ASAN_RT, ASAN_OPTIONS="detect_leaks=0")
    r = subprocess.run([sys.executable, str(script), os.path.join(B.HERE, "_abi.py"), lib],
                       capture_output=True, text=True, timeout=300, env=env)
    assert "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0 and "host checks ok" in r.stdout, (r.stdout, r.stderr[-4000:])
