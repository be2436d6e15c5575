"""Builds libbaretile_amd.so from csrc/*.hip with hipcc for gfx950, in the package directory.

`python -m baretile_amd.build` or build() from Python. The library is one shared object with a C ABI
(include/baretile_amd.h), loaded by baretile_amd._lib with ctypes.
"""
import glob, os, subprocess, sys, tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libbaretile_amd.so")
SOURCES = sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")))
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-shared", "-fPIC",
         # packed fp32 adds and multiplies stay out of the device code (hipcc's host pass warns that it doesn't know
         # the feature, which is harmless)
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-result", "-I", os.path.join(os.path.dirname(HERE), "include")]


def hipcc():
  for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
    if c and (os.path.isabs(c) and os.path.exists(c) or not os.path.isabs(c)): return c
  raise RuntimeError("hipcc not found")


def build(verbose=False):
  """Compile every source into LIB (a temporary name first, so a failed build leaves the old library). The sources
  compile side by side, one hipcc each, then link into one shared object."""
  tmp = LIB + ".tmp"
  cc = hipcc()
  with tempfile.TemporaryDirectory() as work:
    objs = [os.path.join(work, os.path.basename(s)[:-4] + ".o") for s in SOURCES]
    cmds = [[cc, *FLAGS, "-c", "-o", o, s] for s, o in zip(SOURCES, objs)]
    for c in cmds:
      if verbose: print(" ".join(c), flush=True)
    procs = [subprocess.Popen(c, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True) for c in cmds]
    outs = [p.communicate()[0] for p in procs]
    link = [cc, *FLAGS, "-o", tmp, *objs]
    for p, out in zip(procs + [None], outs + [None]):
      if p is None:
        p = subprocess.run(link, capture_output=True, text=True)
        out = p.stdout + p.stderr
      errors = [l for l in out.splitlines() if "packed-fp32-ops" not in l and l.strip()]
      if p.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errors[-60:]))
      if verbose and errors: print("\n".join(errors[-40:]))
  os.replace(tmp, LIB)
  return LIB


if __name__ == "__main__":
  print(build(verbose="-v" in sys.argv))
