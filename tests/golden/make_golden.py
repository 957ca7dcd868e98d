"""Write golden input/output vectors from the reference implementation.

Run in the build container only (the reference checkout is not present on
the GPU box):  ``python tests/golden/make_golden.py /root/reference``.

It imports the reference's own PyTorch code on the CPU for the functions that
no invariant or closed form pins on its own, and stores only data (inputs and
outputs) in ``tests/golden/reference_vectors.npz``:

* ``src/kernels/prescore_selection.py:62-68`` ``_morton_code`` at 10 and 16
  bits -- the fp32 normalise/quantise step whose interior rounding no property
  fixes;
* ``src/kernels/prescore_selection.py:71-84`` ``select_morton_window`` on rows
  whose codes are all distinct (the reference's ``argsort`` is not stable, so
  rows with equal codes have no pinned order and are left out);
* ``src/agents/mappo.py:332-420`` ``AttentionComm.forward`` for the hot-path
  modes, with its weights, so the module composition (qkv split order, gelu,
  projection) is pinned as well as the core;
* ``src/kernels/prescore_selection.py:87-163`` ``grid_knn_shape`` and
  ``select_grid_knn`` -- the cell quantisation, the capacity cut and what a
  query with fewer than k candidates keeps are fixed by that code alone
  (stored as sorted index sets: ``topk(sorted=False)`` leaves the order open).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "reference_vectors.npz"


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from src.agents.mappo import AttentionComm, MAPPOConfig  # noqa: E402
    from src.kernels.prescore_selection import (  # noqa: E402
        _morton_code, grid_knn_shape, select_grid_knn, select_morton_window)

    data: dict[str, np.ndarray] = {}
    g = torch.Generator().manual_seed(20240601)

    # -- Morton codes ------------------------------------------------------
    pos_cases = {
        "m6": torch.rand(3, 6, 2, generator=g) * 2 - 1,
        "m64": torch.rand(2, 64, 2, generator=g),
        "m512": torch.rand(2, 512, 2, generator=g),
        # one agent per integer grid point: exercises exact quantisation edges
        "mgrid": (torch.stack(torch.meshgrid(torch.arange(8.0), torch.arange(8.0),
                                             indexing="ij"), -1).reshape(1, 64, 2) / 7.0),
        # degenerate spans: every agent at one point, and a zero-width axis
        "mflat": torch.full((1, 6, 2), 0.25),
        "mline": torch.stack([torch.linspace(-1, 1, 12), torch.full((12,), 3.0)], -1)[None],
    }
    for name, pos in pos_cases.items():
        pos = pos.float().contiguous()
        data[f"{name}_pos"] = pos.numpy()
        for bits in (10, 16):
            data[f"{name}_code{bits}"] = _morton_code(pos, bits).numpy().astype(np.uint32)

    # -- Morton window (reference fixes bits = 10) -------------------------
    for name in ("m6", "m64", "m512", "mgrid"):
        pos = torch.from_numpy(data[f"{name}_pos"])
        code = _morton_code(pos, 10)
        srt = code.sort(-1).values
        distinct = (srt[:, 1:] != srt[:, :-1]).all(-1).numpy()
        data[f"{name}_distinct10"] = distinct
        for k in (1, 2, 3, 4):
            if k >= pos.shape[1]:
                continue
            data[f"{name}_win{k}"] = select_morton_window(pos, k).numpy().astype(np.int16)

    # -- AttentionComm.forward ----------------------------------------------
    modes = [("dense", 0), ("dense_sdpa", 0), ("topk", 2), ("topk_gather", 1),
             ("topk_gather", 2), ("topk_gather", 3), ("zorder_k", 2), ("zorder_k", 1)]
    for n_agents in (6, 24):
        for msg_dim in (8, 16):
            torch.manual_seed(1000 + 7 * n_agents + msg_dim)
            x = torch.randn(8, n_agents, 32)
            pos = torch.rand(8, n_agents, 2) * 2 - 1
            tag = f"comm_n{n_agents}_d{msg_dim}"
            data[f"{tag}_x"] = x.numpy()
            data[f"{tag}_pos"] = pos.numpy()
            for mode, k in modes:
                torch.manual_seed(77)
                cfg = MAPPOConfig(obs_dim=18, n_actions=5, n_agents=n_agents, hidden=32,
                                  use_comm=True, msg_dim=msg_dim, attn_mode=mode, topk=k)
                mod = AttentionComm(cfg, in_dim=32).eval()
                mod.collect_info = False
                with torch.no_grad():
                    out, _ = mod(x, pos if mode == "zorder_k" else None)
                key = f"{tag}_{mode}_k{k}"
                data[f"{key}_out"] = out.numpy()
                # Same seed and shapes for every mode, so one weight set per tag.
                for pname, p in mod.state_dict().items():
                    if pname.startswith(("qkv.", "proj.")):
                        wkey = f"{tag}_w_{pname}"
                        if wkey in data:
                            assert np.array_equal(data[wkey], p.numpy())
                        data[wkey] = p.numpy()

    # -- grid kNN selector ----------------------------------------------------
    shapes = [(N, k) for N in (6, 48, 96, 192, 384, 512, 1024) for k in (1, 2, 4, 8, 16) if k < N]
    data["grid_shape"] = np.array([(N, k) + tuple(grid_knn_shape(N, k)) for N, k in shapes],
                                  dtype=np.int64)
    gg = torch.Generator().manual_seed(4242)
    cluster = torch.rand(2, 512, 2, generator=gg)
    cluster[:, :200] = 0.45 + 0.1 * cluster[:, :200]      # one crowded area: capacity cut
    cluster[:, 200:203] = torch.tensor([[0.0, 0.0], [1.0, 1.0], [0.0, 1.0]])
    sparse = torch.rand(2, 512, 2, generator=gg) ** 3     # empty corner: short candidate lists
    grid_cases = {
        "g96": (torch.rand(2, 96, 2, generator=gg), (2,)),
        "g192": (torch.rand(2, 192, 2, generator=gg), (2, 4)),
        "g512": (torch.rand(2, 512, 2, generator=gg) * 2 - 1, (2, 4, 8, 16)),
        "gclus": (cluster, (2, 4, 8)),
        "gsparse": (sparse, (2, 4)),
    }
    for name, (pos, ks) in grid_cases.items():
        pos = pos.float().contiguous()
        data[f"{name}_pos"] = pos.numpy()
        for k in ks:
            idx = select_grid_knn(pos, k).sort(-1).values
            data[f"{name}_grid{k}"] = idx.numpy().astype(np.int16)

    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
