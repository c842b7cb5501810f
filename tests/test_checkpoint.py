"""Local FP8 checkpoint loading (CPU) and a loaded block against the oracle (GPU).

The checkpoints here are written by the test: per-expert FP8 tensors with 128x128 block scales
(the naming of FP8 Qwen3-MoE checkpoints), sharded over two files with an index, a single file,
and the already-fused FP8Experts layout.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from oracle import moe_oracle as orc
from tests.helpers import TOL_MAX_ABS, TOL_MEAN_REL, errors, np_f32, to_bf16

E, H, I = 4, 256, 128
P = "model.layers.{}.mlp"


def _f8(rng, shape):
    codes = rng.integers(0, 256, size=shape, dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x3C  # no NaN codes
    return torch.from_numpy(codes).view(torch.float8_e4m3fn)


def _scales(rng, shape):
    return torch.from_numpy(rng.uniform(1e-3, 1e-2, size=shape).astype(np.float32))


def _per_expert(rng, layer):
    t = {f"{P.format(layer)}.gate.weight": torch.from_numpy(rng.normal(0, 0.02, (E, H)).astype(np.float32)).to(torch.bfloat16)}
    for e in range(E):
        base = f"{P.format(layer)}.experts.{e}"
        for proj, shape in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            t[f"{base}.{proj}.weight"] = _f8(rng, shape)
            t[f"{base}.{proj}.weight_scale_inv"] = _scales(rng, (shape[0] // 128, shape[1] // 128))
    return t


def _fused_reference(t, layer):
    """The fused tensors built by hand: experts stacked, gate rows then up rows."""
    p = P.format(layer)
    g = [t[f"{p}.experts.{e}.gate_proj.weight"] for e in range(E)]
    u = [t[f"{p}.experts.{e}.up_proj.weight"] for e in range(E)]
    w13 = torch.stack([torch.cat([g[e], u[e]], 0) for e in range(E)])
    sg = [t[f"{p}.experts.{e}.gate_proj.weight_scale_inv"] for e in range(E)]
    su = [t[f"{p}.experts.{e}.up_proj.weight_scale_inv"] for e in range(E)]
    s13 = torch.stack([torch.cat([sg[e], su[e]], 0) for e in range(E)])
    w2 = torch.stack([t[f"{p}.experts.{e}.down_proj.weight"] for e in range(E)])
    s2 = torch.stack([t[f"{p}.experts.{e}.down_proj.weight_scale_inv"] for e in range(E)])
    return t[f"{p}.gate.weight"], w13, s13, w2, s2


def _write_sharded(tmp_path, tensors):
    names = sorted(tensors)
    half = len(names) // 2
    shards = {"model-00001-of-00002.safetensors": names[:half], "model-00002-of-00002.safetensors": names[half:]}
    wm = {}
    for fn, keys in shards.items():
        save_file({k: tensors[k].contiguous() for k in keys}, os.path.join(tmp_path, fn))
        wm.update({k: fn for k in keys})
    with open(os.path.join(tmp_path, "model.safetensors.index.json"), "w") as fh:
        json.dump({"metadata": {}, "weight_map": wm}, fh)
    return str(tmp_path)


def _same(a, b):
    if a.dtype == torch.float8_e4m3fn:
        return torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    return torch.equal(a, b)


@pytest.fixture()
def ck(pkg):
    import importlib

    return importlib.import_module("inference_server_amd.checkpoint")


def test_sharded_per_expert_checkpoint_fuses_like_transformers(ck, tmp_path):
    rng = np.random.default_rng(0)
    t = {**_per_expert(rng, 0), **_per_expert(rng, 1)}
    path = _write_sharded(tmp_path, t)
    for layer in (0, 1):
        lw = ck.load_moe_layer(path, layer, device="cpu")
        wr, w13, s13, w2, s2 = _fused_reference(t, layer)
        assert lw.fp8
        assert _same(lw.w_router, wr)
        assert _same(lw.gate_up_proj, w13) and _same(lw.gate_up_proj_scale_inv, s13)
        assert _same(lw.down_proj, w2) and _same(lw.down_proj_scale_inv, s2)
        assert lw.gate_up_proj.shape == (E, 2 * I, H) and lw.gate_up_proj_scale_inv.shape == (E, 2 * I // 128, H // 128)


def test_single_file_and_fused_layout(ck, tmp_path):
    rng = np.random.default_rng(1)
    t = _per_expert(rng, 3)
    single = os.path.join(tmp_path, "one.safetensors")
    save_file(t, single)
    a = ck.load_moe_layer(single, 3, device="cpu")
    wr, w13, s13, w2, s2 = _fused_reference(t, 3)
    fused_dir = tmp_path / "fused"
    fused_dir.mkdir()
    p = P.format(3)
    save_file({f"{p}.gate.weight": wr, f"{p}.experts.gate_up_proj": w13, f"{p}.experts.gate_up_proj_scale_inv": s13,
               f"{p}.experts.down_proj": w2, f"{p}.experts.down_proj_scale_inv": s2},
              os.path.join(fused_dir, "model.safetensors"))
    b = ck.load_moe_layer(str(fused_dir), 3, device="cpu")
    for x, y in ((a.gate_up_proj, b.gate_up_proj), (a.gate_up_proj_scale_inv, b.gate_up_proj_scale_inv),
                 (a.down_proj, b.down_proj), (a.down_proj_scale_inv, b.down_proj_scale_inv), (a.w_router, b.w_router)):
        assert _same(x, y)


def test_malformed_checkpoints_fail_loudly(ck, tmp_path):
    rng = np.random.default_rng(2)
    t = _per_expert(rng, 0)
    p = P.format(0)
    missing = {k: v for k, v in t.items() if not k.startswith(f"{p}.experts.3.")}
    d1 = tmp_path / "missing"
    d1.mkdir()
    save_file(missing, os.path.join(d1, "model.safetensors"))
    with pytest.raises(KeyError, match="experts"):
        ck.load_moe_layer(str(d1), 0, device="cpu")
    bad = dict(t)
    bad[f"{p}.experts.1.up_proj.weight_scale_inv"] = _scales(rng, (2, 2))
    d2 = tmp_path / "badscale"
    d2.mkdir()
    save_file(bad, os.path.join(d2, "model.safetensors"))
    with pytest.raises((ValueError, RuntimeError)):
        ck.load_moe_layer(str(d2), 0, device="cpu")
    with pytest.raises(KeyError, match="layers.7"):
        ck.load_moe_layer(str(d2), 7, device="cpu")
    with pytest.raises(FileNotFoundError):
        ck.CheckpointIndex(str(tmp_path / "nothing-here"))


@pytest.mark.gpu
def test_loaded_block_matches_oracle(pkg, ck, dev, tmp_path):
    """A block loaded from a local FP8 checkpoint runs the kernels and matches the oracle."""
    rng = np.random.default_rng(5)
    Eb, Hb, Ib, k, T = 16, 512, 256, 4, 40
    wr = orc.gen_normal_bf16(rng, (Eb, Hb), 0.02)
    w13 = orc.gen_normal_bf16(rng, (Eb, 2 * Ib, Hb), 0.02)
    w2 = orc.gen_normal_bf16(rng, (Eb, Hb, Ib), 0.02)
    q13, s13 = orc.quantize_weight_fp8(w13)
    q2, s2 = orc.quantize_weight_fp8(w2)
    p = P.format(0)
    t = {f"{p}.gate.weight": torch.from_numpy(wr).to(torch.bfloat16)}
    for e in range(Eb):
        t[f"{p}.experts.{e}.gate_proj.weight"] = torch.from_numpy(q13[e, :Ib].copy()).view(torch.float8_e4m3fn)
        t[f"{p}.experts.{e}.up_proj.weight"] = torch.from_numpy(q13[e, Ib:].copy()).view(torch.float8_e4m3fn)
        t[f"{p}.experts.{e}.down_proj.weight"] = torch.from_numpy(q2[e].copy()).view(torch.float8_e4m3fn)
        t[f"{p}.experts.{e}.gate_proj.weight_scale_inv"] = torch.from_numpy(s13[e, :Ib // 128].copy())
        t[f"{p}.experts.{e}.up_proj.weight_scale_inv"] = torch.from_numpy(s13[e, Ib // 128:].copy())
        t[f"{p}.experts.{e}.down_proj.weight_scale_inv"] = torch.from_numpy(s2[e].copy())
    path = _write_sharded(tmp_path, t)
    block = ck.load_moe_block(path, 0, top_k=k, device=dev)
    x = orc.gen_normal_bf16(rng, (T, Hb))
    out = block(to_bf16(x, dev).reshape(1, T, Hb)).reshape(T, Hb)
    # routing from the GPU router's own logits (ties are broken identically), experts by the oracle
    _, w, ids = pkg.route(to_bf16(x, dev), block.gate.weight, k)
    ref = orc.experts_fp8(x, ids.cpu().numpy(), np_f32(w), q13, s13, q2, s2)
    max_abs, mean_rel = errors(np_f32(out), ref)
    assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL
