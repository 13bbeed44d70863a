"""torch-CPU restatement of the vision tower forward (TEST INFRASTRUCTURE ONLY): the CPU baseline
that `bench.py` times on the GPU box's host cores, standing in for the reference's JAX-CPU path
(JAX is not installed there). Same algorithm, cast points and op order as `vision_tower.py`
(which follows /root/reference/model.py:375-388, 540-656, 700-767, 801-851), written with torch's
CPU kernels (MKL/oneDNN GEMMs, the CPU flash-attention kernel) instead of numpy loops, so that it
runs at a speed a CPU user of the reference would see. Full-attention branch only.

Precision: "fp32" (the reference's default dtype; every op in float32) or "bf16" (bf16 storage,
each Dense / rotary / residual op rounding to bf16 as the reference's bf16 mode does; LayerNorm
statistics, GELU and softmax in fp32). Pinned against `vision_tower.encode_vision` in
tests/test_oracle_torch.py.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import indices as ix


def _torch():
    import torch
    return torch


class TorchTower:
    """The tower bound to one Flax-tree param dict, in one precision, on the CPU."""

    def __init__(self, params: Dict, spec, precision: str = "fp32"):
        torch = _torch()
        if precision not in ("fp32", "bf16"):
            raise ValueError(precision)
        self.spec = spec
        self.precision = precision
        self.dt = torch.float32 if precision == "fp32" else torch.bfloat16
        v = params.get("visual", params)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(np.asarray(a, np.float32))).to(self.dt)

        def dense(p):
            return t(p["kernel"]), t(p["bias"])

        def ln(p):
            return t(p["weight"]).float(), t(p["bias"]).float()

        self.patch = dense(v["patch_embed"]["proj"])
        self.pos_table = t(v["pos_embed"]["embedding"]) if spec.num_position_embeddings else None
        self.blocks = []
        for i in range(spec.depth):
            b = v[f"blocks_{i}"]
            self.blocks.append({"norm1": ln(b["norm1"]), "norm2": ln(b["norm2"]), "qkv": dense(b["attn"]["qkv"]),
                                "proj": dense(b["attn"]["proj"]), "fc1": dense(b["mlp"]["linear_fc1"]),
                                "fc2": dense(b["mlp"]["linear_fc2"])})

        def merger(m):
            return {"norm": ln(m["norm"]), "fc1": dense(m["linear_fc1"]), "fc2": dense(m["linear_fc2"])}

        self.merger = merger(v["merger"])
        self.deepstack = [merger(v[f"deepstack_mergers_{j}"]) for j in range(len(spec.deepstack_visual_indexes))]

    # -- ops (each in the tower dtype unless stated) ------------------------------------------
    def _dense(self, x, wb):
        w, b = wb
        return (x @ w) + b          # bf16: the product rounds, then the bias add rounds

    def _ln(self, x, gb):
        g, b = gb
        xf = x.float()
        mean = xf.mean(-1, keepdim=True)
        var = ((xf - mean) ** 2).mean(-1, keepdim=True)
        return ((xf - mean) * _torch().rsqrt(var + 1e-6) * g + b).to(self.dt)

    def _gelu(self, x):
        return _torch().nn.functional.gelu(x.float(), approximate="tanh").to(self.dt)

    @staticmethod
    def _rotate_half(x):
        x1, x2 = x.chunk(2, dim=-1)
        return _torch().cat((-x2, x1), dim=-1)

    def _attention(self, x, blk, cos, sin, cu):
        torch = _torch()
        n = x.shape[0]
        D, H = self.spec.hidden_size, self.spec.num_heads
        hd = D // H
        qkv = self._dense(x, blk["qkv"])
        q, k, v = qkv.split(D, dim=-1)
        q = q.reshape(n, H, hd)
        k = k.reshape(n, H, hd)
        v = v.reshape(n, H, hd)
        q = q * cos + self._rotate_half(q) * sin
        k = k * cos + self._rotate_half(k) * sin
        out = torch.empty((n, H, hd), dtype=self.dt)
        for s, e in zip(cu[:-1], cu[1:]):
            s, e = int(s), int(e)
            if e <= s:
                continue
            qs = q[s:e].transpose(0, 1).float()
            ks = k[s:e].transpose(0, 1).float()
            vs = v[s:e].transpose(0, 1).float()
            o = torch.nn.functional.scaled_dot_product_attention(qs[None], ks[None], vs[None], scale=hd ** -0.5)[0]
            out[s:e] = o.transpose(0, 1).to(self.dt)
        return self._dense(out.reshape(n, D), blk["proj"])

    def block(self, i, x, cos, sin, cu):
        """VisionBlock i (model.py:627-630) on x [N, D] in the tower dtype; cos / sin [N, 1, hd] in the
        tower dtype, cu the segment bounds."""
        blk = self.blocks[i]
        x = x + self._attention(self._ln(x, blk["norm1"]), blk, cos, sin, cu)
        return x + self._dense(self._gelu(self._dense(self._ln(x, blk["norm2"]), blk["fc1"])), blk["fc2"])

    def _merger(self, x, m, postshuffle):
        D4 = 4 * self.spec.hidden_size
        if postshuffle:
            x = self._ln(x.reshape(-1, D4), m["norm"])
        else:
            x = self._ln(x, m["norm"]).reshape(-1, D4)
        return self._dense(self._gelu(self._dense(x, m["fc1"])), m["fc2"])

    def _pos_embed(self, grid):
        torch = _torch()
        idx, wts = ix.pos_embed_taps_ref(grid, self.spec.num_position_embeddings, self.spec.spatial_merge_size)
        w = torch.from_numpy(wts).to(self.dt)
        terms = [self.pos_table[torch.from_numpy(idx[j].astype(np.int64))] * w[j][:, None] for j in range(4)]
        return terms[0] + terms[1] + terms[2] + terms[3]

    def __call__(self, pixel_values, grid_thw) -> Tuple[object, List[object]]:
        """(tokens, deepstack) as torch tensors in the tower dtype (model.py:801-851)."""
        out = self.run(pixel_values, grid_thw)
        return out["tokens"], out["deepstack"]

    def run(self, pixel_values, grid_thw, keep_layers: bool = False) -> Dict[str, object]:
        """The forward with its taps: {"tokens", "deepstack"} and, with keep_layers, "embed" (x after
        the patch embed and pos-embed add) and "layers" (x after each block), torch tensors in the
        tower dtype."""
        torch = _torch()
        grid = np.asarray(grid_thw, np.int64).reshape(-1, 3)
        px = torch.from_numpy(np.ascontiguousarray(pixel_values, np.float32)).to(self.dt)
        out: Dict[str, object] = {}
        with torch.inference_mode():
            x = self._dense(px, self.patch)
            if self.pos_table is not None:
                x = x + self._pos_embed(grid)
            if keep_layers:
                out["embed"] = x.clone()
                out["layers"] = []
            rot = ix.rotary_half_ref(grid, self.spec.hidden_size // self.spec.num_heads, self.spec.spatial_merge_size)
            emb = torch.from_numpy(np.concatenate([rot, rot], axis=-1).astype(np.float32))
            cos, sin = emb.cos().to(self.dt)[:, None, :], emb.sin().to(self.dt)[:, None, :]
            cu = ix.cu_seqlens_ref(grid)
            feats = []
            ds = list(self.spec.deepstack_visual_indexes)
            for i in range(len(self.blocks)):
                x = self.block(i, x, cos, sin, cu)
                if keep_layers:
                    out["layers"].append(x.clone())
                if i in ds:
                    feats.append(self._merger(x, self.deepstack[len(feats)], True))
            out["tokens"] = self._merger(x, self.merger, False)
            out["deepstack"] = feats
        return out
