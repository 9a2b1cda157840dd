"""Build the gfx950 libraries in-tree with hipcc / g++.

  seedvr2_ncnn_amd/lib/libseedvr2_hip.so     HIP kernels + the C-ABI (include/seedvr2_hip.h)
  seedvr2_ncnn_amd/lib/libseedvr2_layers.so  ncnn-surface layers (AdaptiveWindowAttention,
                                             SharedLinear, DecomposedConv3D,
                                             VAEChunkedMHA, VAEDownsample3D,
                                             VAEUpsample3D, the DiT block's norm /
                                             modulation layers) over the C-ABI, the
                                             ncnn-compatible Mat/Layer/Net subset and
                                             the DiT block-graph runner

Every HIP file is compiled for gfx950 only, with packed-fp32 instruction
selection disabled.  Usage: python -m seedvr2_ncnn_amd.build [--force]
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "lib")
INCLUDE = os.path.join(ROOT, "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + INCLUDE, "-I" + CSRC,
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-I" + INCLUDE,
             "-I" + os.path.join(CSRC, "ncnn"), "-I" + os.path.join(CSRC, "layers")]

HIP_SOURCES = ["awa_kernels.hip", "linear_kernels.hip", "pipeline_kernels.hip", "block_kernels.hip",
               "conv3d_kernels.hip", "conv3d_narrow_kernels.hip", "mha_kernels.hip", "graph_ops_kernels.hip", "capi.hip",
               "awa_plan.cpp", "stream_scratch.cpp"]
LAYER_SOURCES = ["ncnn/mat.cpp", "ncnn/layer.cpp", "ncnn/net.cpp", "ncnn/builtin_layers.cpp",
                 "layers/hip_allocator.cpp",
                 "layers/adaptive_window_attention.cpp", "layers/shared_linear.cpp",
                 "layers/decomposed_conv3d.cpp", "layers/vae_chunked_mha.cpp",
                 "layers/vae_resample3d.cpp", "layers/dit_block_ops.cpp",
                 "layers/dit_block_fold.cpp", "layers/dit_block_graph.cpp"]

HIP_LIB = os.path.join(LIB, "libseedvr2_hip.so")
LAYER_LIB = os.path.join(LIB, "libseedvr2_layers.so")


def _headers():
    out = []
    for d, _, files in os.walk(CSRC):
        out += [os.path.join(d, f) for f in files if f.endswith(".h")]
    out += [os.path.join(INCLUDE, f) for f in os.listdir(INCLUDE) if f.endswith(".h")]
    return out


def _stale(target, deps):
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(d) > t for d in deps)


def _obj(src):
    return os.path.join(BUILD, src.replace("/", "_") + ".o")


def _compile(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("compile failed:\n" + " ".join(cmd) + "\n" + err)
    return err


def build(force: bool = False, verbose: bool = False) -> None:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    hdrs = _headers()
    jobs = []
    for src in HIP_SOURCES:
        s = os.path.join(CSRC, src)
        o = _obj(src)
        if force or _stale(o, [s] + hdrs):
            lang = ["-x", "hip"] if src.endswith(".hip") else []
            jobs.append([HIPCC] + HIP_FLAGS + lang + ["-c", s, "-o", o])
    for src in LAYER_SOURCES:
        s = os.path.join(CSRC, src)
        o = _obj(src)
        if force or _stale(o, [s] + hdrs):
            jobs.append(["g++"] + CXX_FLAGS + ["-c", s, "-o", o])
    with cf.ThreadPoolExecutor(max_workers=min(8, max(1, len(jobs)))) as ex:
        for err in ex.map(_compile, jobs):
            if verbose and err.strip():
                print(err, file=sys.stderr)
    hip_objs = [_obj(s) for s in HIP_SOURCES]
    if force or _stale(HIP_LIB, hip_objs):
        _compile([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", HIP_LIB] + hip_objs)
    layer_objs = [_obj(s) for s in LAYER_SOURCES]
    if force or _stale(LAYER_LIB, layer_objs + [HIP_LIB]):
        _compile(["g++", "-shared", "-fPIC", "-o", LAYER_LIB] + layer_objs +
                 ["-L" + LIB, "-lseedvr2_hip", "-Wl,-rpath,$ORIGIN"])


if __name__ == "__main__":
    build(force="--force" in sys.argv, verbose=True)
    print("built", HIP_LIB, LAYER_LIB)
