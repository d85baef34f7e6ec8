"""Write tests/golden/perstep_smaps.npz from the reference's committed result files (data only):

- results/oracle/perstep_batch_sweep.json: the per-step oracle sparsity maps S[7 projections]
  [32 layers] for B in {2,4,8,16,32,64} x 5 groups x 11 decode steps, on a
  0.1 grid, stored here as uint8 tenths, with each group-step's mean sparsity;
- results/kernel/perstep_actual_kernel_speedup.json: the reference's published A100X kernel
  speedups over cuBLAS dense for those maps (per batch size and per group-step).

bench.py --workload perstep replays the maps on this build's kernels.

    python tests/golden/make_perstep_fixture.py   # needs the reference checkout at /root/reference
"""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("REFERENCE_ROOT", "/root/reference")
PROJS = ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"]


def main() -> None:
    sweep = json.load(open(os.path.join(REF, "results/oracle/perstep_batch_sweep.json")))
    speed = json.load(open(os.path.join(REF, "results/kernel/perstep_actual_kernel_speedup.json")))
    rows = [r for r in sweep["rows"] if r.get("record_type") == "group_step"]
    ref_steps = {(int(r["batch_size"]), int(r["group_id"]), int(r["step"])): r for r in speed["step_rows"]}
    keys, maps, mean_s, r_speed, r_dense, r_sparse = [], [], [], [], [], []
    for r in rows:
        b, g, st = int(r["batch_size"]), int(r["group_id"]), int(r["step"])
        k = f"B{b}_g{g}_step{st}"
        if k not in sweep["S"] or (b, g, st) not in ref_steps:
            continue
        m = np.asarray(sweep["S"][k], dtype=np.float64)
        assert m.shape == (len(PROJS), 32)
        tenths = np.rint(m * 10.0)
        assert np.allclose(tenths / 10.0, m, atol=1e-9)
        keys.append((b, g, st))
        maps.append(tenths.astype(np.uint8))
        mean_s.append(float(r["mean_sparsity"]))
        rr = ref_steps[(b, g, st)]
        r_speed.append(float(rr["kernel_speedup"]))
        r_dense.append(float(rr["dense_ms"]))
        r_sparse.append(float(rr["sparse_ms"]))
    keys = np.asarray(keys, dtype=np.int16)
    np.savez_compressed(
        os.path.join(HERE, "perstep_smaps.npz"),
        batch=keys[:, 0], group=keys[:, 1], step=keys[:, 2],
        smap_tenths=np.stack(maps), mean_sparsity=np.asarray(mean_s),
        ref_step_speedup=np.asarray(r_speed), ref_step_dense_ms=np.asarray(r_dense),
        ref_step_sparse_ms=np.asarray(r_sparse),
        ref_batch=np.asarray([int(r["batch_size"]) for r in speed["rows"]], dtype=np.int32),
        ref_batch_speedup=np.asarray([float(r["kernel_speedup"]) for r in speed["rows"]]),
        projs=np.asarray(PROJS),
    )
    print(f"wrote {len(keys)} group-steps")


if __name__ == "__main__":
    main()
