"""Build libsta_hip.so in-tree from csrc/*.hip for gfx950.

    python sparse-thresholded-attention_amd/build.py

hipcc cross-compiles without a GPU.  Every HIP source is compiled with packed-fp32 instruction
selection disabled (-Xclang -target-feature -Xclang -packed-fp32-ops); the host pass warns that
it does not know the feature, which is harmless.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libsta_hip.so")
BUILD = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("STA_OFFLOAD_ARCH", "gfx950")
SOURCES = ["sta_score.hip", "sta_score6.hip", "sta_select.hip", "sta_select_w.hip", "sta_gather.hip", "sta_pq.hip", "sta_stream.hip", "sta_api.hip",
           "sta_dca.hip", "sta_api_pq.hip", "sta_api_stream.hip", "sta_api_dca.hip", "sta_decode.hip",
           "sta_api_decode.hip", "sta_rows.hip", "sta_dca_sel.hip", "sta_dca_dec.hip", "sta_chunk.hip"]
FLAGS = ["--offload-arch=" + ARCH, "-O3", "-fPIC", "-std=c++17", "-Wall",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I" + CSRC, "-I" + os.path.join(os.path.dirname(HERE), "include")]


# per-source code-generation options: the score kernel keeps its MFMA accumulators in VGPRs (its
# epilogue reads them every block) and its Q operands in AGPRs
EXTRA = {"sta_score.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
         "sta_score6.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
         "sta_rows.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _compile(src):
    obj = os.path.join(BUILD, src.replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{msgs}")
    return obj, msgs


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        results = list(ex.map(_compile, SOURCES))
    for _, msgs in results:
        if msgs.strip() and verbose:
            print(msgs, file=sys.stderr)
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp, *[o for o, _ in results]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
