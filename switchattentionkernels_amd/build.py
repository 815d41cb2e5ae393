"""Build libswattn.so in-tree with hipcc for gfx950.

``python -m switchattentionkernels_amd.build`` (or ``__graft_entry__.build()``)
compiles every HIP source under ``csrc/`` into ``libswattn.so`` next to this
file.  The library links against the HIP runtime that PyTorch-ROCm ships
(``torch/lib/libamdhip64.so``) so that one process never holds two HIP
runtimes; stream handles from ``torch.cuda.current_stream().cuda_stream``
are then valid inside the library.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libswattn.so")
ARCH = "gfx950"

SOURCES = ["swattn_index.hip", "swattn_fwd.hip", "swattn_merge.hip", "swattn_decode.hip",
           "swattn_bwd.hip"]
# The measurement probe bench.py uses, in a library of its own (not part of the
# attention library's ABI).
PROBE_SOURCES = ["probe/mfma_probe.hip"]
PROBE_LIB = os.path.join(HERE, "libswattn_probe.so")


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def _torch_lib_dir() -> str | None:
    try:
        import importlib.util
        spec = importlib.util.find_spec("torch")
        if spec is None or spec.origin is None:
            return None
        d = os.path.join(os.path.dirname(spec.origin), "lib")
        return d if os.path.exists(os.path.join(d, "libamdhip64.so")) else None
    except Exception:
        return None


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wno-inline-asm",  # M0 is set and clobbered explicitly by the LDS DMA asm
        "-shared",
        # Keep the compiler from forming packed fp32 instructions.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # MFMA results in ordinary VGPRs: kernels whose registers exceed 256
        # otherwise get every MFMA in the AGPR form, and the VALU then copies
        # each score tile out of (and accumulators back into) AGPRs.
        "-mllvm", "-amdgpu-mfma-vgpr-form=1",
        "-I", os.path.join(ROOT, "include"),
        "-I", CSRC,
    ]


GENERATED = [("gen_fwd_wide.py", "swattn_fwd_wide.inc"), ("gen_bwd_dq.py", "swattn_bwd_dq.inc"),
             ("gen_bwd_dkdv.py", "swattn_bwd_dkdv.inc")]


def generate_sources() -> None:
    """Run the assembly generators under ``csrc/`` (their outputs are
    included by the HIP sources and are not kept in the repository)."""
    for gen, out in GENERATED:
        subprocess.run([sys.executable, os.path.join(CSRC, gen), os.path.join(CSRC, out)], check=True,
                       stdout=subprocess.DEVNULL)


def build(verbose: bool = False, out: str = LIB, extra_flags=(), sources=None) -> str:
    """Compile ``libswattn.so`` (or ``out``, with ``extra_flags`` appended to
    the compile flags; ``sources`` relative to ``csrc/``, default the
    attention library's); returns its path.  Always regenerates the
    generated includes and recompiles."""
    generate_sources()
    cmd = [_hipcc()] + compile_flags() + list(extra_flags)
    tl = _torch_lib_dir()
    if tl is not None:
        cmd += ["-L", tl, "-Wl,-rpath," + tl]
    cmd += [os.path.join(CSRC, s) for s in (SOURCES if sources is None else sources)]
    tmp = out + ".tmp"
    cmd += ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(line for line in res.stderr.splitlines()
                    if "packed-fp32-ops" not in line and line.strip())
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err:
        print(err, file=sys.stderr)
    os.replace(tmp, out)
    return out


def build_probe(verbose: bool = False) -> str:
    """Compile ``libswattn_probe.so`` (bench.py's MFMA-rate probe)."""
    return build(verbose=verbose, out=PROBE_LIB, sources=PROBE_SOURCES)


C_CALLER_SRC = os.path.join(ROOT, "tests", "c_abi", "prefill_caller.cpp")
C_CALLER = os.path.join(ROOT, "tests", "c_abi", "prefill_caller")


def build_c_caller(verbose: bool = False) -> str:
    """Compile the C++ test program that drives ``libswattn.so`` through the
    C ABI alone (``tests/c_abi/prefill_caller``), with no Python or torch in
    its process.  The program and the library then share the one HIP runtime
    (``libamdhip64.so.7``) the loader resolves for it."""
    cmd = [_hipcc(), "-O2", "-std=c++17", "-I", os.path.join(ROOT, "include"), C_CALLER_SRC,
           "-L", HERE, "-Wl,-rpath," + HERE, "-lswattn"]
    tmp = C_CALLER + ".tmp"
    cmd += ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr}")
    os.replace(tmp, C_CALLER)
    return C_CALLER


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_probe(verbose=True))
    print(build_c_caller(verbose=True))
