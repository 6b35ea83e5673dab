"""Builds libbiv_hip.so (the gfx950 MoE backend) in-tree with hipcc.

    python -m biv_amd.build

Flags that the numerics depend on:
  -ffp-contract=off                          no fused multiply-add unless written (fmaf)
  -fhip-fp32-correctly-rounded-divide-sqrt   IEEE f32 division, as the quantiser's amax/127
  -fno-gpu-flush-denormals-to-zero           keep f32 denormals
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-FP32 instructions
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libbiv_hip.so")
SOURCES = ["kernels.hip", "mfma.hip", "api.cpp", "gguf.cpp"]
ARCH = "gfx950"

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def hipcc():
    for p in ("/opt/rocm/bin/hipcc", "hipcc"):
        if os.path.exists(p) or p == "hipcc":
            return p


def build(verbose=False, defines=(), out=OUT):
    """Compiles every source and links `out`.  `defines` (NAME=VALUE) select
    tuning variants of the kernels for measurement; the default build takes
    none."""
    objdir = os.path.join(HERE, "_build" if not defines else "_build_" + "_".join(defines).replace("=", ""))
    os.makedirs(objdir, exist_ok=True)
    def compile_one(src):
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        lang = ["-x", "hip"]
        cmd = [hipcc()] + FLAGS + ["-D" + d for d in defines] + lang + ["-I", os.path.join(ROOT, "include"), "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd))
        r = subprocess.run(cmd, capture_output=True, text=True)
        # hipcc's host pass does not know the packed-fp32 target feature: harmless
        err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{err}")
        if err.strip() and verbose:
            print(err)
        return obj

    # the sources compile independently: one hipcc each, side by side
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", out] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    return out


PROBES = os.path.join(ROOT, "tests", "probes")


def link_flags(src_path):
    """Libraries a probe names on a first line '// probe-links: biv_hip oracle':
    the in-tree libbiv_hip.so and the CPU oracle (test checker), found at run
    time relative to the executable."""
    with open(src_path) as f:
        first = f.readline()
    if not first.startswith("// probe-links:"):
        return []
    libs = first.split(":", 1)[1].split()
    flags = []
    for lib in libs:
        if lib == "biv_hip":
            flags += ["-L", HERE, "-lbiv_hip", "-Wl,-rpath,$ORIGIN/../../biv_amd"]
        elif lib == "oracle":
            sys.path.insert(0, os.path.join(ROOT, "oracle"))
            import oracle
            oracle.build()
            flags += ["-L", os.path.dirname(oracle.LIB_PATH), "-loracle", "-Wl,-rpath,$ORIGIN/../../oracle/_build"]
        else:
            raise RuntimeError(f"{src_path}: unknown probe library {lib}")
    return flags


def build_probes(verbose=False):
    """The GPU test programs under tests/probes (each <name>.cpp, HIP, into
    an executable <name> beside it)."""
    outs = []
    for src in sorted(f for f in os.listdir(PROBES) if f.endswith(".cpp")):
        exe = os.path.join(PROBES, src[:-4])
        cmd = [hipcc()] + FLAGS + ["-x", "hip", os.path.join(PROBES, src), "-o", exe] + \
            link_flags(os.path.join(PROBES, src))
        if verbose:
            print(" ".join(cmd))
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
            raise RuntimeError(f"hipcc failed on {src}:\n{err}")
        outs.append(exe)
    return outs


if __name__ == "__main__":
    # python -m biv_amd.build [-v] [-DNAME=VALUE ... -o PATH]: a variant build
    args = sys.argv[1:]
    defs = [a[2:] for a in args if a.startswith("-D")]
    out = args[args.index("-o") + 1] if "-o" in args else OUT
    print(build(verbose="-v" in args, defines=defs, out=out))
    if not defs:
        print(*build_probes(verbose="-v" in args), sep="\n")
