"""Write golden vectors from the reference implementation (JHollenb/mrun-pub) for the
functions no closed form or published KAT pins bit for bit.

Run once in the build container, where the reference is mounted read-only:
    python tests/golden/make_golden.py /root/reference
It imports the reference's own functions, evaluates them on small seeded inputs and writes
plain ``.npz`` fixtures (arrays only, loaded with ``allow_pickle=False``) plus
``golden_manifest.json`` (SHA-256 per file).  Nothing here runs at test time and the
reference never travels with the fixtures.

Sections (pass their names after the reference root to write only those; default: all):
* ``core``     -- w8a8.npz, codecs.npz, moe.npz
* ``moe_forward`` -- moe_forward.npz: streamed_moe_forward's expert math on a tiny layer
* ``queue``    -- queue.npz: build_expert_queue / build_expert_queue_flat / scatter_committed
* ``page_cache`` -- page_cache.json: the reference's ExpertPageCache (device "cpu") driven
  through seeded random sequences of decode / prefill slot-binding acquires, transient
  prefills and resets, with its whole host state recorded after every call, plus its page
  trace manifest
* ``lowbit_store`` -- lowbit_store/ (an int3 and an int2 store in the reference's layout,
  tests/test_qstore_int3.py:24-56, with an fp32 extras block, an alias and 24-row matmul
  chunks) and lowbit_store.npz: what the reference's QStoreInt3 / QStoreInt2 return for
  them (matmul, matmul_row_stable, embed_rows, fp32)
* ``refstore`` -- refstore/legacy (a store in the reference's own test layout,
  tests/test_qstore_cache.py:19-46) and refstore/v3 (a v3 store sealed by the reference's
  provenance functions), with refstore.npz / refstore.json holding what the reference's
  ``QStore`` returns for them (weight, embed_rows, matmul, identity digests)

Functions covered (reference file:line):
* w8a8_matmul, _int8_gemm              src/mrun/engine/kernels/w8a8.py:33-125
* _quant_row_int3                      src/mrun/engine/kernels/qstore_int3.py:42-56
* _quant_row_int2                      src/mrun/engine/kernels/qstore_int2.py:36-63
* _quant_row_int8                      src/mrun/engine/kernels/qstore_build.py:496-501
* grouped_route_tensors_with_inverse   src/mrun/engine/olmoe_cuda.py:1108-1135 (CPU branch)
* stable_route_reduce                  src/mrun/engine/qwen3_moe_cuda.py:2561-2664 (CPU branch)
* build_expert_queue(_flat), scatter_committed
                                       src/mrun/engine/kernels/expert_queue.py:242-398, 487-514
* streamed_moe_forward (per-expert math) src/mrun/engine/moe_safetensors.py:404, 585-627
* QStore.weight / embed_rows / matmul, _load_qstore_manifest
                                       src/mrun/engine/kernels/qstore.py:326-373, 1026-1128
* ExpertPageCache (slot policy, decode protection, transient-frequency-v1 prefill, the
  mrun-qwen3-moe-page-trace-v1 trace)
                                       src/mrun/engine/qwen3_moe_cuda.py:983-1777
* build_source/builder/derived_provenance
                                       src/mrun/store_provenance.py:86-275, 390-412
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def _write_legacy_store(d: Path, shapes: dict, seed: int) -> None:
    """A qrow-only store in the reference's test layout (no dtype, no schema version, an
    unreferenced 4-byte extras file), written with this script's own code."""
    rng = np.random.default_rng(seed)
    blocks, w_parts, s_parts = {}, [], []
    w_off = s_off = 0
    for name, (out, inn) in shapes.items():
        q = rng.integers(-128, 128, size=(out, inn), dtype=np.int8)
        sc = (rng.random(out) + 0.1).astype(np.float32)
        blocks[name] = {"kind": "qrow", "shape": [out, inn], "w_off": w_off, "w_len": out * inn,
                        "s_off": s_off, "s_len": out * 4}
        w_parts.append(q.reshape(-1))
        s_parts.append(sc)
        w_off += out * inn
        s_off += out * 4
    d.mkdir(parents=True)
    np.concatenate(w_parts).tofile(d / "weights.i8")
    np.concatenate(s_parts).tofile(d / "scales.f32")
    np.zeros(1, np.float32).tofile(d / "extras.f32")
    (d / "manifest.json").write_text(json.dumps({"arch": "qwen2", "config": {"hidden_size": 8}, "blocks": blocks}))


def refstore_section(files: dict) -> None:
    import shutil
    import tempfile

    import torch

    from mrun import store_provenance as sp
    from mrun.engine.kernels import qstore_build as qb
    from mrun.engine.kernels.qstore import QStore

    root = HERE / "refstore"
    if root.exists():
        shutil.rmtree(root)
    root.mkdir()
    arrays: dict = {}
    info: dict = {}

    # legacy store: reference test layout, opened by the reference without validation
    _write_legacy_store(root / "legacy", {"L0.q": (32, 16), "L0.up": (48, 16)}, seed=0)
    st = QStore("legacy", root=root)
    ids = np.array([[3, 0, 31], [7, 7, 1]], dtype=np.int64)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 16)).astype(np.float32)
    arrays["legacy_ids"] = ids
    arrays["legacy_x"] = x
    for name in ("L0.q", "L0.up"):
        arrays[f"legacy_weight_{name}"] = st.weight(name).numpy()
        arrays[f"legacy_embed_{name}"] = st.embed_rows(name, ids).numpy()
        arrays[f"legacy_matmul_{name}"] = st.matmul(name, torch.from_numpy(x)).numpy()
    stb = QStore("legacy", root=root, compute_dtype="bf16")
    arrays["legacy_weight_bf16_L0.up"] = stb.weight("L0.up").float().numpy()
    info["legacy"] = {"identity_status": st.identity_status,
                      "content_identity_verified": bool(st.content_identity_verified)}

    # v3 store: blocks written here, provenance records built by the reference's own
    # functions over a tiny stand-in checkpoint directory, opened (and so verified) by the
    # reference's QStore
    d = root / "v3"
    d.mkdir()
    rng = np.random.default_rng(1)
    blocks = {}
    q0 = rng.integers(-127, 128, size=(24, 32), dtype=np.int8)
    s0 = (rng.uniform(0.5, 1.5, 24) / 127).astype(np.float32)
    q1 = rng.integers(-127, 128, size=(16, 24), dtype=np.int8)
    s1 = (rng.uniform(0.5, 1.5, 16) / 127).astype(np.float32)
    n0 = rng.standard_normal(32).astype(np.float32)
    (d / "weights.i8").write_bytes(q0.tobytes() + q1.tobytes())
    (d / "scales.f32").write_bytes(s0.tobytes() + s1.tobytes())
    (d / "extras.f32").write_bytes(n0.tobytes())
    blocks["L0.gate"] = {"kind": "qrow", "shape": [24, 32], "w_off": 0, "w_len": 768, "s_off": 0, "s_len": 96}
    blocks["L0.down"] = {"kind": "qrow", "shape": [16, 24], "w_off": 768, "w_len": 384, "s_off": 96, "s_len": 64}
    blocks["L0.norm"] = {"kind": "fp32", "shape": [32], "e_off": 0, "e_len": 128}
    blocks["lm_head"] = {"alias": "L0.gate"}
    with tempfile.TemporaryDirectory() as tmp:
        ck = Path(tmp) / "ckpt"
        ck.mkdir()
        (ck / "config.json").write_text(json.dumps({"hidden_size": 32}))
        (ck / "model.safetensors").write_bytes(b"stand-in checkpoint shard")
        source = sp.build_source_provenance(ck, [ck / "model.safetensors"], model_name="tiny-v3",
                                            hf_id="local/tiny-v3", revision="0" * 40)
    builder = sp.build_builder_provenance([Path(qb.__file__)], name="qstore_build",
                                          schema_version=qb.QSTORE_SCHEMA,
                                          quantization=qb.QSTORE_QUANTIZATION)
    manifest = {"schema_version": qb.QSTORE_SCHEMA, "model_name": "tiny-v3", "arch": "qwen2",
                "dtype": "int8", "tie_word_embeddings": False, "config": {"hidden_size": 32},
                "source": source, "builder": builder, "blocks": blocks}
    manifest["derived"] = sp.build_derived_provenance(d, qb.QSTORE_FILES, semantic_manifest=manifest)
    (d / "manifest.json").write_text(json.dumps(manifest, indent=2, sort_keys=True) + "\n")
    st3 = QStore("v3", root=root)
    assert st3.content_identity_verified, st3.identity_status
    info["v3"] = {k: st3.store_identity.get(k) for k in
                  ("identity_status", "content_identity_verified", "source_checkpoint_sha256",
                   "derived_store_sha256", "manifest_semantic_sha256")}
    x3 = np.random.default_rng(9).standard_normal((2, 32)).astype(np.float32)
    arrays["v3_x"] = x3
    arrays["v3_weight_lm_head"] = st3.weight("lm_head").numpy()
    arrays["v3_matmul_L0.gate"] = st3.matmul("L0.gate", torch.from_numpy(x3)).numpy()
    arrays["v3_weight_L0.down"] = st3.weight("L0.down").numpy()
    arrays["v3_fp32_L0.norm"] = st3.fp32("L0.norm").numpy()
    files["refstore.npz"] = arrays
    (HERE / "refstore.json").write_text(json.dumps(info, indent=1, sort_keys=True) + "\n")


def main(ref_root: str, sections: list[str]) -> None:
    sys.path.insert(0, str(Path(ref_root) / "src"))
    files: dict = {}
    if "refstore" in sections:
        refstore_section(files)
    if "core" in sections:
        core_section(files)
    if "queue" in sections:
        queue_section(files)
    if "moe_forward" in sections:
        moe_forward_section(files)
    manifest_path = HERE / "golden_manifest.json"
    manifest = json.loads(manifest_path.read_text()) if manifest_path.exists() else {}
    if "lowbit_store" in sections:
        lowbit_store_section(files)
    if "page_cache" in sections:
        path = page_cache_section()
        manifest[path.name] = hashlib.sha256(path.read_bytes()).hexdigest()
    for name, arrs in files.items():
        path = HERE / name
        np.savez(path, **arrs)
        manifest[name] = hashlib.sha256(path.read_bytes()).hexdigest()
    manifest_path.write_text(json.dumps(manifest, indent=1, sort_keys=True) + "\n")
    print(json.dumps(manifest, indent=1))


def lowbit_store_section(files: dict) -> None:
    import torch

    from mrun.engine.kernels.qstore import QStoreInt2, QStoreInt3
    from mrun.engine.kernels.qstore_int2 import _quant_row_int2
    from mrun.engine.kernels.qstore_int3 import _quant_row_int3

    rng = np.random.default_rng(41)
    root = HERE / "lowbit_store"
    arrays: dict = {}
    x = rng.standard_normal((3, 320)).astype(np.float32)
    ids = np.array([[0, 69, 5], [33, 33, 1]], dtype=np.int64)
    arrays.update(x=x, ids=ids)
    for bits, quant, cls in ((3, _quant_row_int3, QStoreInt3), (2, _quant_row_int2, QStoreInt2)):
        W = rng.standard_normal((70, 320)).astype(np.float32)
        W2 = rng.standard_normal((50, 320)).astype(np.float32)
        p1, s1 = quant(W)
        p2, s2 = quant(W2)
        norm = rng.standard_normal(320).astype(np.float32)
        d = root / f"toy-int{bits}"
        d.mkdir(parents=True, exist_ok=True)
        (d / f"weights.i{bits}").write_bytes(p1.tobytes() + p2.tobytes())
        (d / "scales.f32").write_bytes(s1.tobytes() + s2.tobytes())
        (d / "extras.f32").write_bytes(norm.tobytes())
        blk = lambda p, sc, w_off, s_off, n: {"kind": f"qrow{bits}", "shape": [n, 320], "w_off": w_off,  # noqa: E731
                                             "row_bytes": p.shape[1], "s_off": s_off, "n_groups": sc.shape[1],
                                             "group_size": 128}
        (d / "manifest.json").write_text(json.dumps({
            "model_name": "toy", "arch": "qwen2", "dtype": f"int{bits}", "group_size": 128, "config": {},
            "matmul_chunk_rows": 24,
            "blocks": {"A": blk(p1, s1, 0, 0, 70), "B": blk(p2, s2, p1.nbytes, s1.nbytes, 50),
                       "norm": {"kind": "fp32", "shape": [320], "e_off": 0}, "A2": {"alias": "A"}}}))
        store = cls("toy", root=root)
        t = f"i{bits}"
        xt = torch.from_numpy(x)
        for name in ("A", "B"):
            arrays[f"{t}_{name}_matmul"] = store.matmul(name, xt).numpy()
            arrays[f"{t}_{name}_row_stable"] = store.matmul_row_stable(name, xt).numpy()
        arrays[f"{t}_A2_embed"] = store.embed_rows("A2", ids).numpy()
        arrays[f"{t}_norm"] = store.fp32("norm").numpy()
        store.close()
    files["lowbit_store.npz"] = arrays


def _tiny_fp8_store(root: Path, layers: int, experts: int) -> Path:
    """A packed expert store in the reference's FP8 file format (manifest fields of
    qwen3_moe_cuda.py:780-795), pages filled with a byte pattern, written by this script."""
    from mrun.engine.qwen3_moe_cuda import ExpertPageLayout

    layout = ExpertPageLayout.create(hidden_size=4, intermediate_size=2)
    pages = (np.arange(layout.page_stride, dtype=np.int64)[None, :] + 17 * np.arange(layers * experts)[:, None])
    root.mkdir(parents=True, exist_ok=True)
    (root / "experts.fp8").write_bytes((pages % 256).astype(np.uint8).tobytes())
    (root / "manifest.json").write_text(json.dumps({
        "schema_version": "qwen3-moe-packed-expert-store-v1", "codec": "rowwise-e4m3fn-paged-v1",
        "data_file": "experts.fp8", "layers": layers, "num_experts": experts, "layout": layout.as_dict()}))
    return root


def page_cache_section() -> Path:
    import tempfile

    import torch

    from mrun.engine.qwen3_moe_cuda import ExpertPageCache, PackedFP8ExpertStore

    configs = [
        dict(name="lfu_transient", layers=3, experts=6, max_active=4, capacity=4,
             cache_policy="layer-frequency-lru-v1", prefill="transient-frequency-v1", steps=40, seed=1),
        dict(name="lfu_transient_wide", layers=2, experts=8, max_active=6, capacity=9,
             cache_policy="layer-frequency-lru-v1", prefill="transient-frequency-v1", steps=40, seed=2),
        dict(name="global", layers=3, experts=5, max_active=3, capacity=5,
             cache_policy="global-lru-v1", prefill="cache-fill-v1", steps=30, seed=3),
        dict(name="lfu", layers=4, experts=5, max_active=4, capacity=7,
             cache_policy="layer-frequency-lru-v1", prefill="cache-fill-v1", steps=30, seed=4),
    ]
    out = {"configs": []}
    with tempfile.TemporaryDirectory() as tmp:
        for cfg in configs:
            rng = np.random.default_rng(cfg["seed"])
            store = PackedFP8ExpertStore(_tiny_fp8_store(Path(tmp) / cfg["name"], cfg["layers"], cfg["experts"]))
            stride = store.layout.page_stride
            cache = ExpertPageCache(store, device="cpu", cache_mb=cfg["capacity"] * stride / 1e6,
                                    max_active_pages=cfg["max_active"], cache_policy=cfg["cache_policy"],
                                    page_binding_policy="slot-indirect-v1", prefill_page_policy=cfg["prefill"],
                                    route_prefetch=False, page_trace=True)
            assert cache.capacity == cfg["capacity"]
            ops = []
            for _ in range(cfg["steps"]):
                r = rng.random()
                layer = int(rng.integers(0, cfg["layers"]))
                n_exp = int(rng.integers(1, cfg["max_active"] + 1))
                experts = rng.choice(cfg["experts"], size=n_exp, replace=False)
                routed = [int(e) for e in rng.choice(experts, size=int(rng.integers(n_exp, 3 * n_exp + 1)))]
                routed += [int(e) for e in experts]  # every chosen expert is routed at least once
                rng.shuffle(routed)
                idx = torch.tensor([routed])
                if r < 0.05:
                    clear = bool(rng.random() < 0.5)
                    cache.reset(clear_pages=clear)
                    op = {"op": "reset", "clear_pages": clear}
                elif r < 0.40 and cfg["prefill"] == "transient-frequency-v1":
                    sel, _, gs = cache.acquire_transient_prefill(layer, idx)
                    op = {"op": "transient", "layer": layer, "routed": routed, "selected": sel.tolist(),
                          "group_slots": gs.tolist()}
                else:
                    protect = bool(rng.random() < 0.6)
                    sel, _, slots = cache.acquire_slot_binding(layer, idx, protect=protect)
                    op = {"op": "acquire", "layer": layer, "routed": routed, "protect": protect,
                          "selected": sel.tolist(), "slots": slots.tolist()}
                op["entries"] = [[k[0], k[1], int(v)] for k, v in cache.entries.items()]
                op["decode_protected"] = sorted([list(k) for k in cache.decode_protected])
                op["layer_entry_counts"] = list(cache.layer_entry_counts)
                op["free_slots"] = list(cache.free_slots)
                stats = cache.stats.as_dict()
                op["stats"] = [stats[k] for k in sorted(stats)]
                ops.append(op)
            out["configs"].append({**cfg, "page_stride": stride, "ops": ops, "stats_keys": sorted(stats),
                                   "trace": cache.export_page_trace(), "trace_status": cache.page_trace_status()})
    path = HERE / "page_cache.json"
    path.write_text(json.dumps(out, sort_keys=True) + "\n")
    return path


def core_section(files: dict) -> None:
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


def queue_section(files: dict) -> None:
    import torch

    from mrun.engine.kernels.expert_queue import build_expert_queue, build_expert_queue_flat, scatter_committed

    rng = np.random.default_rng(31)
    arrays: dict = {}
    rows, E, k, H = 40, 24, 6, 20
    top = np.stack([rng.permutation(E)[:k] for _ in range(rows)]).astype(np.int64)
    w = rng.random((rows, k)).astype(np.float32)
    ep = rng.integers(0, 5, size=rows).astype(np.int64)
    dl = rng.integers(100, 200, size=rows).astype(np.int64)
    arrays.update(d_top=top, d_w=w, d_ep=ep, d_dl=dl)
    for tag, tw in (("f32", torch.from_numpy(w)), ("bf16", torch.from_numpy(w).to(torch.bfloat16))):
        plan = build_expert_queue(torch.from_numpy(top), tw, num_experts=E, epochs=torch.from_numpy(ep),
                                  deadlines=torch.from_numpy(dl))
        for f in ("token_ids", "expert_ids", "route_slots", "coefficients", "epochs", "deadlines", "starts", "counts"):
            arrays[f"d_{tag}_{f}"] = getattr(plan, f).numpy()
        out = rng.standard_normal((plan.assignments, H)).astype(np.float32)
        active = np.where(rng.random(rows) < 0.7, ep, ep + 1).astype(np.int64)
        red, valid = scatter_committed(plan, torch.from_numpy(out), active_epochs=torch.from_numpy(active))
        arrays[f"d_{tag}_out"], arrays[f"d_{tag}_active"] = out, active
        arrays[f"d_{tag}_reduced"], arrays[f"d_{tag}_valid"] = red.numpy(), valid.numpy()
    # pruned packets: a random subset of the dense (row, slot) pairs, in a shuffled order
    keep = rng.random(rows * k) < 0.6
    tok = np.repeat(np.arange(rows), k)[keep]
    slot = np.tile(np.arange(k), rows)[keep]
    exp = top.reshape(-1)[keep]
    cf = w.reshape(-1)[keep]
    perm = rng.permutation(tok.size)
    tok, slot, exp, cf = tok[perm], slot[perm], exp[perm], cf[perm]
    plan = build_expert_queue_flat(torch.from_numpy(tok), torch.from_numpy(exp), torch.from_numpy(slot),
                                   torch.from_numpy(cf), num_rows=rows, num_experts=E, top_k=k,
                                   epochs=torch.from_numpy(ep), deadlines=torch.from_numpy(dl))
    arrays.update(f_tok=tok, f_slot=slot, f_exp=exp, f_cf=cf)
    for f in ("token_ids", "expert_ids", "route_slots", "coefficients", "epochs", "deadlines", "starts", "counts"):
        arrays[f"f_{f}"] = getattr(plan, f).numpy()
    out = rng.standard_normal((plan.assignments, H)).astype(np.float32) * 3
    active = np.where(rng.random(rows) < 0.5, ep, ep - 1).astype(np.int64)
    red, valid = scatter_committed(plan, torch.from_numpy(out), active_epochs=torch.from_numpy(active))
    arrays.update(f_out=out, f_active=active, f_reduced=red.numpy(), f_valid=valid.numpy())
    files["queue.npz"] = arrays


def moe_forward_section(files: dict) -> None:
    """streamed_moe_forward on a tiny 2-layer Qwen3-MoE whose layer-0 experts hold int8
    codes x row scales exactly; layer 0's attention is ablated (an exact zero contribution),
    so the residual after layer 0 is h0 + moe(rmsnorm(h0))."""
    import tempfile

    import torch
    import transformers

    from mrun.engine.moe_safetensors import PagedSafetensors, _rmsnorm, streamed_moe_forward

    rng = np.random.default_rng(41)
    E, k, H, I, T = 8, 3, 32, 24, 12
    cfg = transformers.Qwen3MoeConfig(
        vocab_size=99, hidden_size=H, intermediate_size=48, moe_intermediate_size=I, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=2, head_dim=8, num_experts=E, num_experts_per_tok=k,
        norm_topk_prob=True, decoder_sparse_step=1, max_position_embeddings=64, attn_implementation="eager",
        tie_word_embeddings=False)
    torch.manual_seed(0)
    model = transformers.Qwen3MoeForCausalLM(cfg).eval().float()
    gu_q = rng.integers(-127, 128, size=(E, 2 * I, H), dtype=np.int8)
    gu_s = (rng.uniform(0.5, 1.5, size=(E, 2 * I)) / 127 / np.sqrt(H)).astype(np.float32)
    dn_q = rng.integers(-127, 128, size=(E, H, I), dtype=np.int8)
    dn_s = (rng.uniform(0.5, 1.5, size=(E, H)) / 127 / np.sqrt(I)).astype(np.float32)
    router = rng.standard_normal((E, H)).astype(np.float32)
    ln = rng.uniform(0.5, 1.5, size=H).astype(np.float32)
    layer = model.model.layers[0]
    with torch.no_grad():
        layer.mlp.experts.gate_up_proj.copy_(torch.from_numpy(gu_q.astype(np.float32) * gu_s[..., None]))
        layer.mlp.experts.down_proj.copy_(torch.from_numpy(dn_q.astype(np.float32) * dn_s[..., None]))
        layer.mlp.gate.weight.copy_(torch.from_numpy(router))
        layer.post_attention_layernorm.weight.copy_(torch.from_numpy(ln))
        model.model.embed_tokens.weight.copy_(torch.from_numpy(rng.standard_normal((99, H)).astype(np.float32)))
    ids = rng.integers(1, 99, size=T)
    arrays = dict(gu_q=gu_q, gu_s=gu_s, dn_q=dn_q, dn_s=dn_s, router=router, ln=ln, ids=ids)
    eps = float(cfg.rms_norm_eps)
    with tempfile.TemporaryDirectory() as tmp:
        d = Path(tmp) / "m"
        model.save_pretrained(str(d), safe_serialization=True)
        cfg.save_pretrained(str(d))
        ps = PagedSafetensors(d)
        for tag, dt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
            got = streamed_moe_forward(ps, torch.from_numpy(ids), dtype=dt, capture_hidden_states=True,
                                       ablate_component=(0, "attn"), skip_lm_head=True)
            h0, h1 = got["hidden_states"][0], got["hidden_states"][1]
            y = _rmsnorm(h0.to(dt), torch.from_numpy(ln).to(dt), eps)
            arrays[f"{tag}_h0"] = h0.float().numpy()
            arrays[f"{tag}_h1"] = h1.float().numpy()
            arrays[f"{tag}_y"] = y.float().numpy()
            arrays[f"{tag}_top_idx"] = got["topk_idx"][0].astype(np.int64)
            arrays[f"{tag}_top_w"] = got["topk_w"][0].astype(np.float32)
    files["moe_forward.npz"] = arrays


SECTIONS = ("core", "refstore", "queue", "moe_forward", "page_cache", "lowbit_store")

if __name__ == "__main__":
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    main(root, sys.argv[2:] or list(SECTIONS))
