#!/usr/bin/env python3
"""Write the golden vectors of the DCA prefill (dual-chunk positions, dense attention).

Run ONCE in the build container (the reference repository is read-only at /root/reference and
never travels to a GPU box):

    python tests/golden/gen_golden_dca.py

The reference's DCA core is the prefill branch of the attention forward that
_make_dca_forward builds (dca_kernel.py:372-489), with the position tables of
ChunkLlamaRotaryEmbedding (:166-231) and the PyTorch attention path of _fa_block (:292-349;
flash_attn is not installed here) merged by _merge_lse (:352-366).  It is executed here on a
minimal attention module whose projections are exact slices (q, k and v are passed through
unchanged) and whose output projection is the identity, so the recorded output is exactly the
attention core's.  Cases cover all three position types, GQA, mscale above the pretraining
length, fp32 and bf16 model dtypes.
"""
import math
import os
import sys
from types import SimpleNamespace

import numpy as np
import torch

REF = "/root/reference"
OUT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, OUT)
from gen_golden import planted_inputs  # noqa: E402


def _import_reference():
    sys.path.insert(0, REF)
    import dca_kernel as dca  # noqa: E402
    return dca


class _Core(torch.nn.Module):
    """Attention module whose projections hand q, k and v through unchanged."""

    def __init__(self, dca, H, Hkv, D, pretrain_len, dtype):
        super().__init__()
        self.head_dim, self.num_heads, self.num_key_value_heads, self.layer_idx = D, H, Hkv, 0
        self.config = SimpleNamespace(num_attention_heads=H, num_key_value_heads=Hkv)
        self.scaling = D ** -0.5
        width = (H + 2 * Hkv) * D
        eye = torch.eye(width, dtype=dtype)
        self.q_proj = torch.nn.Linear(width, H * D, bias=False, dtype=dtype)
        self.k_proj = torch.nn.Linear(width, Hkv * D, bias=False, dtype=dtype)
        self.v_proj = torch.nn.Linear(width, Hkv * D, bias=False, dtype=dtype)
        self.o_proj = torch.nn.Linear(H * D, H * D, bias=False, dtype=dtype)
        with torch.no_grad():
            self.q_proj.weight.copy_(eye[:H * D])
            self.k_proj.weight.copy_(eye[H * D:(H + Hkv) * D])
            self.v_proj.weight.copy_(eye[(H + Hkv) * D:])
            self.o_proj.weight.copy_(torch.eye(H * D, dtype=dtype))
        self.rotary_emb = dca.ChunkLlamaRotaryEmbedding(dim=D, max_position_embeddings=pretrain_len, base=10000)


def gen(dca):
    cases = [
        # chunk_size s, pretrain c, local w -> chunk_len L = s - w
        dict(name="three_types_gqa_fp32", H=2, Hkv=1, N=300, D=64, s=96, c=128, w=32, dtype=torch.float32, seed=51),
        dict(name="three_types_bf16", H=2, Hkv=2, N=400, D=64, s=160, c=192, w=32, dtype=torch.bfloat16, seed=52),
        dict(name="intra_only_fp32", H=1, Hkv=1, N=120, D=64, s=160, c=192, w=32, dtype=torch.float32, seed=53),
        dict(name="d128_bf16", H=2, Hkv=1, N=330, D=128, s=96, c=256, w=32, dtype=torch.bfloat16, seed=54),
    ]
    arrays = {}
    with torch.no_grad():
        for i, c in enumerate(cases):
            dca._DCA_CHUNK_SIZE, dca._DCA_LOCAL_WINDOW = c["s"], c["w"]
            core = _Core(dca, c["H"], c["Hkv"], c["D"], c["c"], c["dtype"])
            q, k, v = planted_inputs(c["seed"], c["H"], c["Hkv"], c["N"], c["D"], 0.02, c["dtype"])
            hidden = torch.cat([q[0].transpose(0, 1).reshape(c["N"], -1), k[0].transpose(0, 1).reshape(c["N"], -1),
                                v[0].transpose(0, 1).reshape(c["N"], -1)], dim=-1)[None]
            fwd = dca._make_dca_forward(c["s"], c["c"], c["w"])
            out, _ = fwd(core, hidden, None, None, None)
            out = out[0].reshape(c["N"], c["H"], c["D"]).transpose(0, 1).contiguous()
            p = f"c{i}_"
            store = (lambda t: t.view(torch.int16).numpy().view(np.uint16)) if c["dtype"] == torch.bfloat16 \
                else (lambda t: t.numpy())
            arrays[p + "q"], arrays[p + "k"], arrays[p + "v"] = store(q[0]), store(k[0]), store(v[0])
            arrays[p + "out"] = out.float().numpy()
            arrays[p + "params"] = np.array([c["s"], c["c"], c["w"], 1 if c["dtype"] == torch.bfloat16 else 0],
                                            np.int64)
            mscale = dca.get_mscale(c["N"] / c["c"])
            print(f"dca case {i} {c['name']}: L={c['s'] - c['w']} chunks={math.ceil(c['N'] / (c['s'] - c['w']))} "
                  f"mscale={mscale:.6f}", flush=True)
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(OUT, "dca_golden.npz"), **arrays)


if __name__ == "__main__":
    torch.set_num_threads(8)
    gen(_import_reference())
