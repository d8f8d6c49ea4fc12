"""Write golden vectors from the reference implementation (JHollenb/mrun-pub) for the
functions no closed form or published KAT pins bit for bit.

Run once in the build container, where the reference is mounted read-only:
    python tests/golden/make_golden.py /root/reference
It imports the reference's own functions, evaluates them on small seeded inputs and writes
plain ``.npz`` fixtures (arrays only, loaded with ``allow_pickle=False``) plus
``golden_manifest.json`` (SHA-256 per file).  Nothing here runs at test time and the
reference never travels with the fixtures.

Functions covered (reference file:line):
* w8a8_matmul, _int8_gemm              src/mrun/engine/kernels/w8a8.py:33-125
* _quant_row_int3                      src/mrun/engine/kernels/qstore_int3.py:42-56
* _quant_row_int2                      src/mrun/engine/kernels/qstore_int2.py:36-63
* _quant_row_int8                      src/mrun/engine/kernels/qstore_build.py:496-501
* grouped_route_tensors_with_inverse   src/mrun/engine/olmoe_cuda.py:1108-1135 (CPU branch)
* stable_route_reduce                  src/mrun/engine/qwen3_moe_cuda.py:2561-2664 (CPU branch)
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def main(ref_root: str) -> None:
    sys.path.insert(0, str(Path(ref_root) / "src"))
    import torch

    from mrun.engine.kernels.qstore_build import _quant_row_int8
    from mrun.engine.kernels.qstore_int2 import _quant_row_int2
    from mrun.engine.kernels.qstore_int3 import _quant_row_int3
    from mrun.engine.kernels.w8a8 import _int8_gemm, w8a8_matmul
    from mrun.engine.olmoe_cuda import grouped_route_tensors_with_inverse
    from mrun.engine.qwen3_moe_cuda import stable_route_reduce

    files = {}

    # ---- W8A8 -----------------------------------------------------------------------------
    rng = np.random.default_rng(2024)
    out, inn, T = 96, 256, 7
    q_w = rng.integers(-127, 128, size=(out, inn), dtype=np.int8)
    sc_w = (rng.random(out) * 0.02 + 1e-3).astype(np.float32)
    x = rng.standard_normal((T, inn)).astype(np.float32)
    x[:, rng.permutation(inn)[:3]] *= 300.0
    x[0, :5] = [0.0, 1.5, -2.5, 0.25, 0.0]  # halfway ties after scaling are likely
    tq, ts, tx = torch.from_numpy(q_w), torch.from_numpy(sc_w), torch.from_numpy(x)
    arrays = {"q_w": q_w, "sc_w": sc_w, "x": x}
    for k in (0, 4, 8):
        arrays[f"y_k{k}"] = w8a8_matmul(tq, ts, tx, protect_k=k, use_int_mm=False).numpy()
    pidx = np.array([3, 17, 200], dtype=np.int64)
    arrays["protect_idx"] = pidx
    arrays["y_static"] = w8a8_matmul(tq, ts, tx, protect_idx=torch.from_numpy(pidx), use_int_mm=False).numpy()
    qx = rng.integers(-128, 128, size=(9, 200), dtype=np.int8)
    qw = rng.integers(-128, 128, size=(33, 200), dtype=np.int8)
    arrays["gemm_qx"], arrays["gemm_qw"] = qx, qw
    arrays["gemm_acc"] = _int8_gemm(torch.from_numpy(qx), torch.from_numpy(qw), use_int_mm=False).numpy()
    files["w8a8.npz"] = arrays

    # ---- codecs ---------------------------------------------------------------------------
    rng = np.random.default_rng(7)
    W = rng.standard_normal((12, 300)).astype(np.float32)
    W[0, :8] = [1.0, 0.5, -0.5, 1.5, 3.0, -3.0, 0.0, 2.5]  # exact multiples -> ties
    W[1] = 0.0
    W[2, :128] = 0.7  # a constant group (int2 threshold edge: |x| == 0.7 * mean)
    arrays = {"W": W}
    p3, s3 = _quant_row_int3(W)
    p2, s2 = _quant_row_int2(W)
    p3g, s3g = _quant_row_int3(W, G=4)
    p2g, s2g = _quant_row_int2(W, G=4)
    q8, s8 = _quant_row_int8(W)
    arrays.update(p3=p3, s3=s3, p2=p2, s2=s2, p3g4=p3g, s3g4=s3g, p2g4=p2g, s2g4=s2g, q8=q8, s8=s8)
    files["codecs.npz"] = arrays

    # ---- MoE route + reduce ---------------------------------------------------------------
    rng = np.random.default_rng(11)
    Tm, E, k, H = 50, 16, 4, 24
    top = np.stack([rng.permutation(E)[:k] for _ in range(Tm)]).astype(np.int64)
    w32 = rng.random((Tm, k)).astype(np.float32)
    arrays = {"top": top, "w32": w32}
    ti = torch.from_numpy(top)
    for tag, tw in (("f32", torch.from_numpy(w32)), ("bf16", torch.from_numpy(w32).to(torch.bfloat16))):
        tok, coef, starts, counts, inv, _ = grouped_route_tensors_with_inverse(ti, tw, num_experts=E)
        arrays[f"tok_{tag}"] = tok.numpy()
        arrays[f"coef_{tag}"] = coef.float().numpy()
        arrays[f"starts_{tag}"] = starts.numpy()
        arrays[f"counts_{tag}"] = counts.numpy()
        arrays[f"inv_{tag}"] = inv.numpy()
    tok, coef, starts, counts, inv, _ = grouped_route_tensors_with_inverse(ti, torch.from_numpy(w32), num_experts=E)
    eo32 = rng.standard_normal((Tm * k, H)).astype(np.float32)
    sel = torch.arange(E)
    arrays["eo32"] = eo32
    arrays["red_f32"] = stable_route_reduce(torch.from_numpy(eo32), coef, tok, counts, ti, sel, inverse_assignments=inv).numpy()
    eob = torch.from_numpy(eo32).to(torch.bfloat16)
    arrays["eo_bf16_as_f32"] = eob.float().numpy()
    arrays["red_bf16"] = stable_route_reduce(eob, coef.to(torch.bfloat16), tok, counts, ti, sel).numpy()
    files["moe.npz"] = arrays

    manifest = {}
    for name, arrs in files.items():
        path = HERE / name
        np.savez(path, **arrs)
        manifest[name] = hashlib.sha256(path.read_bytes()).hexdigest()
    (HERE / "golden_manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
