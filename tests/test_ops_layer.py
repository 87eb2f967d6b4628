"""Drop-in boundary on the CPU: ops factory, layouts, state-dict loading,
loader nodes, LoRA attach and the PyTorch forward paths, driven through a
minimal ComfyUI stand-in (tests/fake_comfy).

The PyTorch paths are the reference fallback (_ops.py:483-491, :538-545),
so their outputs are checked against the oracle's restatement of it."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import __graft_entry__
import oracle
from _layers import int4_layer, int8_layer, load_linear, write_model

pkg = __graft_entry__.load_package()
ops_mod = __graft_entry__._submodule("_ops")
layout = __graft_entry__._submodule("quant_layout")
loaders = __graft_entry__._submodule("_loaders")


def test_node_mappings_match_reference_signatures():
    m = pkg.NODE_CLASS_MAPPINGS
    assert set(m) == {"SimpleINT4UNetLoader", "SimpleINT8UNetLoader", "IntCrushLoRALoader", "IntCrushLoRAUnloader"}
    for name in ("SimpleINT4UNetLoader", "SimpleINT8UNetLoader"):
        it = m[name].INPUT_TYPES()["required"]
        assert set(it) == {"unet_name", "rot_size"}
        assert it["rot_size"][0] == [0, 16, 64, 256, 1024, 4096] and it["rot_size"][1]["default"] == 256
        assert m[name].RETURN_TYPES == ("MODEL",) and m[name].FUNCTION == "load"
    lo = m["IntCrushLoRALoader"].INPUT_TYPES()["required"]
    assert set(lo) == {"model", "lora_name", "strength"}
    assert (lo["strength"][1]["min"], lo["strength"][1]["max"]) == (-10.0, 10.0)
    assert m["IntCrushLoRAUnloader"].FUNCTION == "unload"
    assert set(pkg.NODE_DISPLAY_NAME_MAPPINGS) == set(m)


def test_layouts_registered_with_comfy():
    import comfy.quant_ops as qo

    assert qo.get_layout_class("IntCrushInt4Layout") is layout.IntCrushInt4Layout
    assert qo.QUANT_ALGOS["int4_crush"]["storage_t"] == torch.uint8
    assert qo.QUANT_ALGOS["int8_crush"]["comfy_tensor_layout"] == "IntCrushInt8Layout"


def test_ops_factory_is_memoised():
    a = ops_mod.make_intcrush_ops("int4_crush", 256)
    assert a is ops_mod.make_intcrush_ops("int4_crush", 256)
    assert a is not ops_mod.make_intcrush_ops("int4_crush", 256, use_w4a16=True)
    for cls in ("Linear", "GroupNorm", "LayerNorm", "Conv2d", "Conv3d", "ConvTranspose2d", "Embedding"):
        assert hasattr(a, cls)


@pytest.mark.parametrize("name,expect", [
    ("double_blocks.0.img_attn.qkv", True), ("single_blocks.3.linear2", True),
    ("single_blocks.3.modulation.lin", False), ("final_layer.adaLN_modulation.1", False),
    ("txt_in.norm", False), ("proj_out", False), ("time_in.embedder", False),
])
def test_rotation_rule_by_layer_name(name, expect):
    ops = ops_mod.make_intcrush_ops("int4_crush", 64)
    lin = load_linear(ops, name, int4_layer(16, 256, seed=1), 256, 16)
    assert lin._intcrush_rot_need is expect
    assert lin._intcrush_is_quantized and lin.quant_format == "int4_crush"
    assert lin._intcrush_w_in == 256


def test_state_dict_load_attributes():
    ops = ops_mod.make_intcrush_ops("int4_crush", 256)
    sd = int4_layer(32, 512, seed=2, zp=True, svd_rank=4)
    lin = load_linear(ops, "blk.fc", sd, 512, 32)
    w = lin.weight
    assert tuple(w._qdata.shape) == (32, 256) and w._qdata.dtype == torch.uint8
    assert w._params.scale.dtype == torch.float32 and tuple(w._params.scale.shape) == (32, 4)
    assert torch.equal(lin._intcrush_perm, sd["weight_perm"])
    assert lin._intcrush_smoothrot_factors.dtype == torch.float32
    assert lin._intcrush_L1.dtype == torch.float16 and lin.bias is not None
    assert hasattr(lin, "weight_perm") and hasattr(lin, "weight_zp")
    ops8 = ops_mod.make_intcrush_ops("int8_crush", 0)
    lin8 = load_linear(ops8, "blk.fc8", int8_layer(32, 256, seed=3), 256, 32)
    assert tuple(lin8.weight._params.scale.shape) == (32,)
    assert lin8.weight._qdata.dtype == torch.int8


def test_non_intcrush_layer_uses_default_loader():
    ops = ops_mod.make_intcrush_ops("int8_crush", 0)
    lin = ops.Linear(8, 4)
    sd = {"p.weight": torch.randn(4, 8), "p.bias": torch.randn(4)}
    lin._load_from_state_dict(sd, "p.", {}, True, [], [], [])
    assert not lin._intcrush_is_quantized
    x = torch.randn(3, 8)
    assert torch.allclose(lin(x), x @ sd["p.weight"].t() + sd["p.bias"])


def test_int4_dequantize_group_layout():
    sd = int4_layer(8, 384, G=3, seed=4, perm=False, smoothrot=False)
    P = layout.IntCrushInt4Layout.Params(scale=sd["weight_scale"].float(), orig_dtype=torch.float16,
                                         orig_shape=(8, 384))
    W = layout.IntCrushInt4Layout.dequantize(sd["weight"], P)
    q = oracle.unpack_int4(sd["weight"].numpy(), 384).astype(np.float32)
    s = sd["weight_scale"].float().numpy()
    ref = q * np.repeat(s, 128, axis=1)
    assert np.array_equal(W.numpy(), ref)


def test_layout_quantize_roundtrip():
    W = torch.randn(16, 64)
    packed, P = layout.IntCrushInt4Layout.quantize(W)
    back = layout.IntCrushInt4Layout.dequantize(packed, P)
    assert (back - W).abs().max() <= P.scale.max() / 2 + 1e-6
    q8, P8 = layout.IntCrushInt8Layout.quantize(W)
    assert (layout.IntCrushInt8Layout.dequantize(q8, P8) - W).abs().max() <= P8.scale.max() / 2 + 1e-6


@pytest.mark.parametrize("G", [1, 4])
def test_cpu_int4_forward_is_reference_fallback(G):
    """CPU tensors take the reference PyTorch path: fp32 dequant -> F.linear
    on the prepared activation, no bias (_ops.py:483-491)."""
    K, N, R = 512, 48, 64
    ops = ops_mod.make_intcrush_ops("int4_crush", R)
    sd = int4_layer(N, K, G=G, seed=5)
    lin = load_linear(ops, "blk.fc", sd, K, N)
    x = torch.randn(2, 5, K)
    out = lin(x)
    assert out.shape == (2, 5, N) and out.dtype == x.dtype
    ref = oracle.reference_fallback_forward(x, sd["weight"].numpy(), sd["weight_scale"].float().numpy(), K,
                                            int4=True, smoothrot=sd["weight_smoothrot_factors"], rot_size=R,
                                            perm=sd["weight_perm"])
    assert torch.allclose(out.reshape(-1, N), ref, rtol=1e-4, atol=1e-4)


def test_cpu_int8_forward_dequant_linear():
    K, N = 256, 40
    ops = ops_mod.make_intcrush_ops("int8_crush", 0)
    sd = int8_layer(N, K, seed=6, smooth=True)
    lin = load_linear(ops, "blk.fc", sd, K, N)
    x = torch.randn(7, K, dtype=torch.bfloat16)
    out = lin(x)
    xs = (x / sd["weight_smooth"].to(torch.bfloat16))
    W = (sd["weight"].to(torch.bfloat16) * sd["weight_scale"].float().reshape(-1, 1).to(torch.bfloat16))
    ref = torch.nn.functional.linear(xs, W, sd["bias"].to(torch.bfloat16))
    assert torch.equal(out, ref)


def test_zero_point_fallback():
    K, N = 256, 16
    ops = ops_mod.make_intcrush_ops("int4_crush", 0, use_pytorch=True)
    sd = int4_layer(N, K, G=2, seed=7, perm=False, smoothrot=False, zp=True)
    lin = load_linear(ops, "blk.fc", sd, K, N)
    x = torch.randn(3, K)
    q = torch.from_numpy(oracle.unpack_int4(sd["weight"].numpy(), K)).float()
    s = sd["weight_scale"].float().repeat_interleave(K // 2, dim=1)
    W = (q - sd["weight_zp"].reshape(-1, 1)) * s
    assert torch.allclose(lin(x), x @ W.t(), rtol=1e-5, atol=1e-5)


def _setup_files(tmp_path, fmt: str):
    import folder_paths

    folder_paths.ROOTS["diffusion_models"] = str(tmp_path / "dm")
    folder_paths.ROOTS["loras"] = str(tmp_path / "loras")
    K, N = 256, 32
    if fmt == "int4":
        layers = {
            "double_blocks.0.img_attn.qkv": (int4_layer(N, K, seed=10), K),
            "single_blocks.0.modulation.lin": (int4_layer(N, K, seed=11, perm=False, smoothrot=False), K),
        }
        meta = {"int_crush.format_version": "3", "int_crush.rot_size": "64"}
    else:
        layers = {
            "double_blocks.0.img_mlp.0": (int8_layer(N, K, seed=12), K),
            "img_in": (int8_layer(N, K + 64, seed=13), K + 64),
        }
        meta = {"int_crush.format_version": "1", "int_crush.rot_size": "0",
                "int_crush.padded_layers": f"img_in.weight={K}"}
    write_model(str(tmp_path / "dm" / f"model_{fmt}.safetensors"), layers, meta)
    return layers


def test_int4_loader_node_reads_metadata(tmp_path):
    layers = _setup_files(tmp_path, "int4")
    (model,) = loaders.SimpleINT4UNetLoader().load("model_int4.safetensors", 256)
    qkv = model.model.double_blocks._modules["0"].img_attn.qkv
    mod = model.model.single_blocks._modules["0"].modulation.lin
    assert qkv._intcrush_rot_size == 64 and qkv._intcrush_rot_need
    assert not mod._intcrush_rot_need
    x = torch.randn(3, 256)
    sd = layers["double_blocks.0.img_attn.qkv"][0]
    ref = oracle.reference_fallback_forward(x, sd["weight"].numpy(), sd["weight_scale"].float().numpy(), 256,
                                            int4=True, smoothrot=sd["weight_smoothrot_factors"], rot_size=64,
                                            perm=sd["weight_perm"])
    assert torch.allclose(qkv(x), ref, rtol=1e-4, atol=1e-4)


def test_int4_loader_rot0_selects_w4a16(tmp_path):
    _setup_files(tmp_path, "int4")
    import safetensors.torch as st

    p = tmp_path / "dm" / "model_int4.safetensors"
    sd = st.load_file(str(p))
    st.save_file(sd, str(tmp_path / "dm" / "plain.safetensors"), metadata={})
    (model,) = loaders.SimpleINT4UNetLoader().load("plain.safetensors", 0)
    qkv = model.model.double_blocks._modules["0"].img_attn.qkv
    assert qkv._intcrush_use_w4a16 and not qkv._intcrush_rot_need


def test_int8_loader_trims_padded_layers(tmp_path):
    _setup_files(tmp_path, "int8")
    (model,) = loaders.SimpleINT8UNetLoader().load("model_int8.safetensors", 256)
    img_in = model.model.img_in
    assert tuple(img_in.weight._qdata.shape) == (32, 256)
    assert img_in.weight._params.orig_shape == (32, 256)
    assert model.model.double_blocks._modules["0"].img_mlp._modules["0"]._intcrush_rot_size == 0


def test_detect_rot_size_rules():
    f = loaders._detect_rot_size
    assert f(None, 256, ("2", "3")) == 256
    assert f({"int_crush.format_version": "3", "int_crush.rot_size": "1024"}, 256, ("2", "3")) == 1024
    assert f({"int_crush.format_version": "1", "int_crush.rot_size": "1024"}, 256, ("2", "3")) == 256
    assert f({"int_crush.format_version": "3", "int_crush.rot_size": "32"}, 64, ("2", "3")) == 64
    assert f({"int_crush.format_version": "3"}, 16, ("2", "3")) == 16


def test_lora_nodes_attach_and_clear(tmp_path):
    from safetensors.torch import save_file

    _setup_files(tmp_path, "int4")
    (model,) = loaders.SimpleINT4UNetLoader().load("model_int4.safetensors", 256)
    qkv = model.model.double_blocks._modules["0"].img_attn.qkv
    x = torch.randn(4, 256)
    base = qkv(x)
    g = torch.Generator().manual_seed(20)
    down, up = torch.randn(8, 256, generator=g) * 0.1, torch.randn(32, 8, generator=g) * 0.1
    (tmp_path / "loras").mkdir(exist_ok=True)
    save_file({"double_blocks.0.img_attn.qkv.lora_down.weight": down,
               "double_blocks.0.img_attn.qkv.lora_up.weight": up,
               "double_blocks.0.img_attn.qkv.alpha": torch.tensor(4.0)}, str(tmp_path / "loras" / "l.safetensors"))
    (model2,) = loaders.IntCrushLoRALoader().load(model, "l.safetensors", 0.5)
    out = qkv(x)
    ref = base + (x @ down.t()) @ up.t() * (4.0 / 8 * 0.5)
    assert torch.allclose(out, ref, rtol=1e-4, atol=1e-4)
    loaders.IntCrushLoRAUnloader().unload(model2)
    assert torch.allclose(qkv(x), base)


def test_casting_hooks_are_used_and_released():
    import comfy.ops as co

    ops = ops_mod.make_intcrush_ops("int4_crush", 0, use_pytorch=True)
    lin = load_linear(ops, "blk.fc", int4_layer(16, 128, seed=21, perm=False, smoothrot=False), 128, 16)
    lin.comfy_cast_weights = True
    co.CAST_CALLS.clear()
    lin(torch.randn(2, 128))
    assert [c[0] for c in co.CAST_CALLS] == ["cast", "uncast"]


# ------------------------------------------------------------------ checkpoint round trip
ckpt = __graft_entry__._submodule("_checkpoint")


def test_padded_layers_format_round_trip():
    d = {"img_in.weight": 64, "blocks.3.ffn.2.weight": 13824}
    s = ckpt.format_padded_layers(d)
    assert s == "img_in.weight=64;blocks.3.ffn.2.weight=13824"
    assert ckpt.parse_padded_layers(s) == d
    assert ckpt.parse_padded_layers("a.weight=5;junk; b.weight = 7 ") == {"a.weight": 5, "b.weight": 7}
    for bad in ({"img_in": 64}, {"a;b.weight": 3}, {"a.weight": 0}):
        with pytest.raises(ValueError):
            ckpt.format_padded_layers(bad)


def test_checkpoint_round_trip_int4(tmp_path):
    """Every tensor of an INT4 checkpoint (packed weights, group scales,
    perm, SmoothRot factors, zero point, SVD factors) and its metadata come
    back bit for bit, and the INT4 loader node reads the saved rot size."""
    import folder_paths

    folder_paths.ROOTS["diffusion_models"] = str(tmp_path / "dm")
    K, N = 256, 32
    layers = {"double_blocks.0.img_attn.qkv": (int4_layer(N, K, G=2, seed=30, zp=True, svd_rank=4), K),
              "single_blocks.0.modulation.lin": (int4_layer(N, K, seed=31, perm=False, smoothrot=False), K)}
    sd = {}
    for name, (lsd, in_f) in layers.items():
        sd.update({f"{name}.{k}": v for k, v in lsd.items()})
        sd[f"__in__.{name}.weight"] = torch.tensor([in_f])  # the stand-in loader's in_features
    path = str(tmp_path / "dm" / "rt4.safetensors")
    meta = ckpt.save_checkpoint(path, sd, rot_size=64, extra_metadata={"note": "test"})
    assert meta == {"int_crush.format_version": "3", "int_crush.rot_size": "64", "note": "test"}
    back, info = ckpt.load_checkpoint(path)
    assert set(back) == set(sd) and all(torch.equal(back[k], sd[k]) and back[k].dtype == sd[k].dtype for k in sd)
    assert (info.fmt, info.format_version, info.rot_size, info.padded_layers) == ("int4_crush", "3", 64, {})
    (model,) = loaders.SimpleINT4UNetLoader().load("rt4.safetensors", 256)
    qkv = model.model.double_blocks._modules["0"].img_attn.qkv
    assert qkv._intcrush_rot_size == 64 and qkv.weight._params.zp is not None
    x = torch.randn(3, K)
    lsd = layers["double_blocks.0.img_attn.qkv"][0]
    assert torch.equal(qkv.weight._qdata, lsd["weight"])
    assert torch.isfinite(qkv(x)).all()


def test_checkpoint_round_trip_int8_padded(tmp_path):
    """An INT8 checkpoint with a padded layer: the metadata round-trips and
    the INT8 loader trims the layer back to its original width."""
    import folder_paths

    folder_paths.ROOTS["diffusion_models"] = str(tmp_path / "dm")
    K, N = 256, 32
    sd = {f"double_blocks.0.img_mlp.0.{k}": v for k, v in int8_layer(N, K, seed=32).items()}
    sd.update({f"img_in.{k}": v for k, v in int8_layer(N, K + 64, seed=33).items()})
    path = str(tmp_path / "dm" / "rt8.safetensors")
    ckpt.save_checkpoint(path, sd, rot_size=0, padded_layers={"img_in.weight": K})
    back, info = ckpt.load_checkpoint(path)
    assert all(torch.equal(back[k], sd[k]) for k in sd)
    assert (info.fmt, info.rot_size, info.padded_layers) == ("int8_crush", 0, {"img_in.weight": K})
    (model,) = loaders.SimpleINT8UNetLoader().load("rt8.safetensors", 256)
    assert tuple(model.model.img_in.weight._qdata.shape) == (N, K)
    assert torch.equal(model.model.img_in.weight._qdata, sd["img_in.weight"][:, :K])


def test_checkpoint_save_rejects_bad_input(tmp_path):
    sd = {f"fc.{k}": v for k, v in int8_layer(8, 64, seed=34).items()}
    p = str(tmp_path / "x.safetensors")
    with pytest.raises(ValueError, match="rot_size"):
        ckpt.save_checkpoint(p, sd, rot_size=128)
    with pytest.raises(KeyError):
        ckpt.save_checkpoint(p, sd, rot_size=0, padded_layers={"other.weight": 32})
    with pytest.raises(ValueError, match="below the stored"):
        ckpt.save_checkpoint(p, sd, rot_size=0, padded_layers={"fc.weight": 64})
    with pytest.raises(ValueError, match="weight format"):
        ckpt.save_checkpoint(p, {"a": torch.zeros(2)}, rot_size=0)
    with pytest.raises(ValueError, match="unknown weight format"):
        ckpt.save_checkpoint(p, sd, rot_size=0, fmt="int2")
    assert not os.path.exists(p)
    # a file without INT-Crush metadata reads as such
    from safetensors.torch import save_file

    save_file({"a": torch.zeros(2)}, p)
    _, info = ckpt.load_checkpoint(p)
    assert (info.fmt, info.rot_size, info.padded_layers) == (None, None, {})


@pytest.mark.parametrize("K_w,G,zp,svd,expect", [
    (3072, 24, False, False, 3072),  # already a multiple of 128
    (64, 1, False, False, 128),      # Flux img_in: per-row scales
    (96, 3, False, False, 128),      # groups of 32: lcm(128, 32) = 128
    (320, 10, False, False, 384),
    (192, 2, False, False, 384),     # groups of 96: lcm(128, 96) = 384
    (100, 1, False, False, 128),
    (80, 5, False, False, 80),       # groups of 16: no MFMA width holds them
    (64, 1, True, False, 64),        # zero point: corrections over the prepared width
    (64, 1, False, True, 64),        # SVD residual: the same
])
def test_gemm_width_of_narrow_layers(K_w, G, zp, svd, expect):
    """The width the drop-in Linear runs the GEMMs at: K_w, or for widths that
    are not a multiple of 128 the next multiple of lcm(128, group size)."""
    from types import SimpleNamespace

    ops_mod = __graft_entry__._submodule("_ops")
    N = 8
    scale = torch.ones(N, G) if G > 1 else torch.ones(N)
    params = SimpleNamespace(scale=scale, zp=torch.zeros(N) if zp else None)
    layer = SimpleNamespace(_intcrush_w_in=K_w, weight=SimpleNamespace(_params=params),
                            _intcrush_L1=torch.zeros(4, K_w) if svd else None)
    assert ops_mod._gemm_width(layer) == expect
