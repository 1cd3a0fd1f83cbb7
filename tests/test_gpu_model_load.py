"""A whole model loaded from an artifact directory and config.json
(sparkmv_model_load: tools/vq-runtime/src/model.rs:121-185 Weights::load
over VqDir, tools/vq/gpu/vq-model-gpu.cu:230-357, :739-775 load_model).

The directory is written here in the reference's layout (manifest.txt, one
RQVQ container or RQVF sidecar per tensor, the reference's tensor names) for
the small model of test_gpu_forward.py with a VQ tied embedding. The loaded
model must give the same logits, bit for bit, as one assembled by hand from
the same bytes, and meet the oracle's 1e-5 (f32 activations). Refusals carry
the reference's messages. A trusted profile in the directory is applied.
"""
import json
import struct

import numpy as np
import pytest

from test_gpu_forward import CFG, FULL, TOKENS, rel_l2

pytestmark = pytest.mark.gpu


def hf_config(c, full):
    return {"hidden_size": c["hidden"], "num_hidden_layers": c["layers"], "num_attention_heads": c["heads"],
            "num_key_value_heads": c["kv_heads"], "head_dim": c["head_dim"], "intermediate_size": c["intermediate"],
            "vocab_size": c["vocab"], "rms_norm_eps": c["eps"], "sliding_window": c["sliding_window"],
            "layer_types": ["full_attention" if f else "sliding_attention" for f in full],
            "rope_parameters": {"full_attention": {"rope_theta": c["rope_full_theta"],
                                                   "partial_rotary_factor": c["rope_full_partial"]},
                                "sliding_attention": {"rope_theta": c["rope_slide_theta"],
                                                      "partial_rotary_factor": c["rope_slide_partial"]}}}


def write_artifact(sm, d, c, overrides=None):
    """Containers, sidecars, manifest.txt and config.json; returns the host
    tensors by name."""
    overrides = overrides or {}
    hd, heads, kvh, hid, inter = c["head_dim"], c["heads"], c["kv_heads"], c["hidden"], c["intermediate"]
    qd, kvd = heads * hd, kvh * hd
    rng = np.random.default_rng(21)
    tensors = {"model.embedding.weight": sm.synth_container(301, c["vocab"], hid),
               "model.norm.weight": (1 + 0.2 * rng.standard_normal(hid)).astype(np.float32)}
    shapes = {"self_attn.q_k_v_proj.weight": (qd + 2 * kvd, hid), "self_attn.g_proj.weight": (heads, hid),
              "self_attn.out_proj.weight": (hid, qd), "mlp.gate_proj.weight": (inter, hid),
              "mlp.up_proj.weight": (inter, hid), "mlp.down_proj.weight": (hid, inter)}
    for li in range(c["layers"]):
        p = f"model.layers.{li}."
        for k, (name, (r, cc)) in enumerate(shapes.items()):
            tensors[p + name] = sm.synth_container(400 + 10 * li + k, r, cc)
        for name in ("input_layernorm.weight", "post_attention_layernorm.weight"):
            tensors[p + name] = (1 + 0.2 * rng.standard_normal(hid)).astype(np.float32)
    tensors.update(overrides)
    lines = ["# name rows cols stages file_bytes relL2"]
    for name, t in tensors.items():
        if t.dtype == np.float32:
            b = b"RQVF" + struct.pack("<II", 1, t.size) + t.tobytes()
            lines.append(f"{name} 1 {t.size} 0 {len(b)} 0")
        else:
            b = t.tobytes()
            h = sm.Container(t)
            lines.append(f"{name} {h.rows} {h.cols} {h.nstages} {len(b)} 0.001")
        (d / f"{name}.bin").write_bytes(b)
    (d / "manifest.txt").write_text("\n".join(lines) + "\n")
    (d / "config.json").write_text(json.dumps(hf_config(c, FULL)))
    return tensors


def by_hand(sm, ref, dev, c, tensors):
    """The same weights assembled in Python, and the oracle over them."""
    import torch

    import forward as fw
    layers, host_layers = [], []
    for li in range(c["layers"]):
        p = f"model.layers.{li}."
        dl, hl = {}, {}
        for key, name in (("qkv", "self_attn.q_k_v_proj.weight"), ("attn_gate", "self_attn.g_proj.weight"),
                          ("out", "self_attn.out_proj.weight"), ("gate", "mlp.gate_proj.weight"),
                          ("up", "mlp.up_proj.weight"), ("down", "mlp.down_proj.weight")):
            dl[key] = sm.DeviceContainer(tensors[p + name], dev)
            hl[key] = ref.decode(tensors[p + name])
        for key, name in (("in_norm", "input_layernorm.weight"), ("post_norm", "post_attention_layernorm.weight")):
            hl[key] = tensors[p + name]
            dl[key] = torch.from_numpy(tensors[p + name]).to(dev)
        dl["full"] = hl["full"] = FULL[li]
        layers.append(dl)
        host_layers.append(hl)
    head = sm.DeviceContainer(tensors["model.embedding.weight"], dev)
    norm = tensors["model.norm.weight"]
    cfg = dict(c, x_dtype=sm.X_F32, dim=4, nc=4096, nstages=2, v3=1)
    model = sm.Model(cfg, layers, head, torch.from_numpy(norm).to(dev))
    oracle = fw.Forward(c, host_layers, ref.decode(tensors["model.embedding.weight"]).astype(np.float32), norm)
    return model, oracle


def test_load_matches_hand_assembled_and_oracle(sm, ref, dev, tmp_path):
    import torch
    c = CFG
    tensors = write_artifact(sm, tmp_path, c)
    loaded = sm.Model.load(tmp_path, tmp_path / "config.json", c["max_ctx"], sm.X_F32)
    hand, oracle = by_hand(sm, ref, dev, c, tensors)
    a = torch.full((c["vocab"],), float("nan"), device=dev)
    b = torch.full((c["vocab"],), float("nan"), device=dev)
    for pos, tok in enumerate(TOKENS):
        loaded.forward(tok, pos, a)
        hand.forward(tok, pos, b)
        torch.cuda.synchronize()
        assert torch.equal(a, b), pos
        err = rel_l2(a.cpu().numpy(), oracle.forward(tok, pos))
        print(f"loaded model pos {pos}: relL2 {err:.2e}")
        assert err <= 1e-5
    del loaded   # frees the weights it uploaded


def test_load_refusals(sm, ref, dev, tmp_path):
    c = CFG
    # a matrix of the wrong shape
    bad = sm.synth_container(77, 48, c["hidden"])
    write_artifact(sm, tmp_path, c, {"model.layers.1.self_attn.g_proj.weight": bad})
    with pytest.raises(sm.SparkmvError, match=r"model.layers.1.self_attn.g_proj.weight: is 48x256, "
                                               r"the architecture needs 4x256"):
        sm.Model.load(tmp_path, tmp_path / "config.json", c["max_ctx"], sm.X_F32)
    # a norm of the wrong width
    write_artifact(sm, tmp_path, c, {"model.layers.2.input_layernorm.weight": np.ones(100, np.float32)})
    with pytest.raises(sm.SparkmvError, match="layer 2: a norm is not 256 wide"):
        sm.Model.load(tmp_path, tmp_path / "config.json", c["max_ctx"], sm.X_F32)
    write_artifact(sm, tmp_path, c, {"model.norm.weight": np.ones(7, np.float32)})
    with pytest.raises(sm.SparkmvError, match="model.norm.weight: 7 values"):
        sm.Model.load(tmp_path, tmp_path / "config.json", c["max_ctx"], sm.X_F32)
    # a matrix of another VQ geometry than the embedding's
    odd = sm.synth_container(78, c["intermediate"], c["hidden"], 4, 1024, 2, 1)
    write_artifact(sm, tmp_path, c, {"model.layers.0.mlp.up_proj.weight": odd})
    with pytest.raises(sm.SparkmvError, match="one model runs one VQ geometry"):
        sm.Model.load(tmp_path, tmp_path / "config.json", c["max_ctx"], sm.X_F32)
    # a tensor the manifest does not list
    write_artifact(sm, tmp_path, c)
    lines = [ln for ln in (tmp_path / "manifest.txt").read_text().splitlines() if "layers.2.mlp.down" not in ln]
    (tmp_path / "manifest.txt").write_text("\n".join(lines) + "\n")
    with pytest.raises(sm.SparkmvError, match="is not in the manifest"):
        sm.Model.load(tmp_path, tmp_path / "config.json", c["max_ctx"], sm.X_F32)


def test_load_applies_a_trusted_profile(sm, ref, dev, tmp_path):
    """A trusted profile is applied at load. As in the reference's runtime
    (vq-model-gpu.cu:1097-1120), a profile that is absent, unreadable or for
    another device never fails the load: the heuristic stays, and the note
    says why."""
    c = CFG
    write_artifact(sm, tmp_path, c)
    hid, qd = c["hidden"], c["heads"] * c["head_dim"]
    cfg_path = tmp_path / "config.json"
    e = sm.ProfileEntry(kind=0, dim=4, nc=4096, rows=hid, cols=qd, v3=1, variant=1, threads=256, rate=1.0)
    fp = sm.profile_fingerprint(tmp_path)
    prof = tmp_path / "vq-tune.profile"
    m = sm.Model.load(tmp_path, cfg_path, c["max_ctx"], sm.X_F32)
    assert m.matvec_kernel(hid, qd) == (0, 0) and "absent" in m.profile_note
    sm.profile_write(prof, fp, sm.device_name(), "hip", [e])
    m = sm.Model.load(tmp_path, cfg_path, c["max_ctx"], sm.X_F32)
    assert m.matvec_kernel(hid, qd) == (1, 256)
    assert "1 geometries take their tuned kernel" in m.profile_note
    m2 = sm.Model.load(tmp_path, cfg_path, c["max_ctx"], sm.X_F32, apply_profile=False)
    assert m2.matvec_kernel(hid, qd) == (0, 0) and "not requested" in m2.profile_note
    sm.profile_write(prof, fp, "some other device", "hip", [e])
    m3 = sm.Model.load(tmp_path, cfg_path, c["max_ctx"], sm.X_F32)
    assert m3.matvec_kernel(hid, qd) == (0, 0) and "another artifact or device" in m3.profile_note
    prof.write_text("VQPROF 7\n")
    m4 = sm.Model.load(tmp_path, cfg_path, c["max_ctx"], sm.X_F32)
    assert m4.matvec_kernel(hid, qd) == (0, 0) and "not version 1" in m4.profile_note
