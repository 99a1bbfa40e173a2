"""Builds libkt_gfx950.so in-tree with hipcc (gfx950 only): each source compiled in parallel, then linked.
`python -m kindi_amd.build`."""
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libkt_gfx950.so")
SOURCES = ["kt_decode.hip", "kt_gemv.hip", "kt_gemv2.hip", "kt_mma.hip", "kt_prefill.hip", "kt_prefill8.hip",
           "kt_moe.hip", "kt_moe1.hip", "kt_fold.hip", "kt_api.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
         # packed fp32 (v_pk_*_f32) stays off: hand-written kernels here use scalar fp32 only
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _clean(out):
    return "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l and "hip-link" not in l)


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    return r.returncode, _clean(r.stdout + r.stderr)


def build(verbose=False, extra=()):
    tmp = tempfile.mkdtemp(prefix="kt_build_")
    objs = [os.path.join(tmp, s.replace(".hip", ".o")) for s in SOURCES]
    cmds = [[HIPCC] + FLAGS + list(extra) + ["-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)]
    with ThreadPoolExecutor(len(cmds)) as ex:
        res = list(ex.map(_run, cmds))
    for (rc, msg), s in zip(res, SOURCES):
        if rc:
            raise RuntimeError("hipcc failed on %s:\n%s" % (s, msg))
        if verbose and msg.strip():
            print(msg)
    rc, msg = _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + objs + ["-o", OUT + ".tmp"])
    if rc:
        raise RuntimeError("link failed:\n" + msg)
    os.replace(OUT + ".tmp", OUT)
    for o in objs:
        os.remove(o)
    os.rmdir(tmp)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
