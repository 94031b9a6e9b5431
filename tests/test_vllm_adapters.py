"""The vLLM-facing surface without vLLM (it is not importable in this image): the quantisation config's checkpoint
scan and per-layer decisions (the reference's config.py:33-133), the linear and MoE methods' loaders and checks
(linear.py:45-99, moe.py:82-122) on stand-in layers, and the plugin's patches of vLLM classes (__init__.py:12-112)
on stand-in classes and modules. The GPU side of the methods (apply) is tests/test_gpu_adapters.py.
"""
import gc
import json
import sys
import types

import pytest
import torch

import vllm_espalier as P
from vllm_espalier import config as C
from vllm_espalier import linear as Lin
from vllm_espalier import moe as Moe
from vllm_espalier import ops
from vllm_espalier import workloads as WL


def test_text_key():
    assert C.text_key("model.layers.3.self_attn.q_proj") == "layers.3.self_attn.q_proj"
    assert C.text_key("model.language_model.layers.0.mlp.experts.7.up_proj") == "layers.0.mlp.experts.7.up_proj"
    assert C.text_key("mtp.layers.0.mlp.gate_proj") == "mtp.layers.0.mlp.gate_proj"       # its own namespace
    assert C.text_key("model.mtp.layers.0.mlp.gate_proj") == "mtp.layers.0.mlp.gate_proj"
    assert C.text_key("lm_head") == "lm_head" and C.text_key("model.lm_head") == "lm_head"
    assert C.text_key("model.visual.blocks.0.attn.qkv") is None
    assert C.text_key("model.embed_tokens") is None


def _weight_map():
    keys = []
    for m in ("q_proj", "k_proj", "v_proj", "o_proj"):
        keys.append(f"model.layers.0.self_attn.{m}.esp_trellis")
        keys.append(f"model.layers.0.self_attn.{m}.suh")
    for e in range(4):
        for p in ("gate_proj", "up_proj", "down_proj"):
            keys.append(f"model.layers.0.mlp.experts.{e}.{p}.esp_trellis")
    for p in ("gate_proj", "up_proj", "down_proj"):
        keys.append(f"model.layers.0.mlp.shared_expert.{p}.esp_trellis")
    keys += ["model.layers.0.mlp.gate.weight", "model.layers.1.self_attn.q_proj.esp_trellis",
             "model.layers.1.self_attn.k_proj.weight", "model.layers.1.self_attn.v_proj.weight",
             "lm_head.esp_trellis", "model.visual.blocks.0.attn.qkv.esp_trellis", "model.norm.weight"]
    return {k: "model-00001.safetensors" for k in keys}


@pytest.fixture
def cfg(tmp_path):
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": _weight_map()}))
    c = C.EspalierConfig.from_config({"quant_method": "Espalier", "bits": 4})
    c.maybe_update_config(str(tmp_path))
    return c


def test_scan_and_layer_decisions(cfg):
    assert cfg.is_exl3("model.layers.0.self_attn.qkv_proj")
    assert cfg.is_exl3("model.layers.0.self_attn.o_proj")
    assert cfg.is_exl3("model.layers.0.mlp.shared_expert.gate_up_proj")
    assert cfg.is_exl3("model.layers.0.mlp.shared_expert.down_proj")
    assert not cfg.is_exl3("model.layers.0.mlp.gate")                    # the router stays unquantised
    assert not cfg.is_exl3("model.visual.blocks.0.attn.qkv")             # the vision tower too
    with pytest.raises(ValueError, match="partly"):
        cfg.is_exl3("model.layers.1.self_attn.qkv_proj")                 # q coded, k / v not
    assert cfg.experts_exl3("model.layers.0.mlp.experts")
    assert not cfg.experts_exl3("model.layers.2.mlp.experts")
    assert cfg.is_exl3("lm_head")
    assert "visual" not in " ".join(cfg.coded)


def test_config_surface(tmp_path):
    with pytest.raises(ValueError):
        C.EspalierConfig.from_config({"quant_method": "gptq"})
    assert C.EspalierConfig.override_quantization_method({"quant_method": "ESPALIER"}, None) == "espalier"
    assert C.EspalierConfig.override_quantization_method({"quant_method": "awq"}, None) is None
    assert C.EspalierConfig.override_quantization_method(None, None) is None
    c = C.EspalierConfig({})
    assert c.get_name() == "espalier" and c.get_min_capability() == 80 and c.get_config_filenames() == []
    assert c.get_supported_act_dtypes() == [torch.bfloat16, torch.float16]
    assert c.packed_modules_mapping["qkv_proj"] == ["q_proj", "k_proj", "v_proj"]
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"a.weight": "x"}}))
    with pytest.raises(ValueError, match="no .esp_trellis"):
        c.maybe_update_config(str(tmp_path))


# stand-ins named as vLLM's layer classes (the config recognises kinds by class name)
class LinearBase(torch.nn.Module):
    pass


class ColumnParallelLinear(LinearBase):
    pass


class ParallelLMHead(torch.nn.Module):
    pass


class RoutedExperts(torch.nn.Module):
    moe_config = None


def test_get_quant_method(cfg):
    assert isinstance(cfg.get_quant_method(ColumnParallelLinear(), "model.layers.0.self_attn.qkv_proj"),
                      Lin.EspLinearMethod)
    assert cfg.get_quant_method(ColumnParallelLinear(), "model.layers.0.mlp.gate") is None   # unquantised
    assert isinstance(cfg.get_quant_method(RoutedExperts(), "model.layers.0.mlp.experts"), Moe.EspMoEMethod)
    with pytest.raises(ValueError, match="routed experts"):
        cfg.get_quant_method(RoutedExperts(), "model.layers.5.mlp.experts")
    assert isinstance(cfg.get_quant_method(ParallelLMHead(), "lm_head"), Lin.EspLinearMethod)
    assert cfg.get_quant_method(torch.nn.LayerNorm(4), "model.norm") is None


def test_shard_order():
    assert [Lin.shard_order(s) for s in (None, "q", "k", "v", 3, (2, 5), [4, 1])] == [0, 0, 1, 2, 3, 2, 1]


def _load_linear(method, layer, shards, gen, K=256):
    for shard, n in shards:
        for suffix, t in WL.matrix_tensors(K, n, 4, "int6", gen).items():
            p = getattr(layer, suffix)
            p.weight_loader(p, t, shard)


def test_linear_loader_orders_shards_and_registers():
    layer = torch.nn.Module()
    method = Lin.EspLinearMethod("model.layers.0.self_attn.qkv_proj")
    method.create_weights(layer, 256, [256, 128, 128], 256, 512, torch.bfloat16)
    gen = torch.Generator().manual_seed(0)
    want = {}
    for shard, n in (("v", 128), ("q", 256), ("k", 128)):                # arrival order is not shard order
        t = WL.matrix_tensors(256, n, 4, "int6", gen)
        want[shard] = t["esp_trellis"]
        for suffix, v in t.items():
            p = getattr(layer, suffix)
            p.weight_loader(p, v, shard)
    method.process_weights_after_loading(layer)
    assert [m.out_features for m in layer.espalier.mats] == [256, 128, 128]
    for i, s in enumerate("qkv"):
        assert torch.equal(layer.espalier.mats[i].trellis, want[s])
        assert getattr(layer.espalier, f"trellis_{i}") is layer.espalier.mats[i].trellis
    assert [n for n, _ in layer.espalier.named_buffers()][:3] == ["trellis_0", "suh_0", "svh_0"]
    assert layer.espalier.state_dict() == {}                             # buffers, not checkpoint state
    key = layer.espalier.dense_key
    assert key is not None and ops.DENSE_LAYERS[key].N == 512 and ops.DENSE_LAYERS[key].K == 256
    assert layer.espalier.pad == 0
    del layer, p                                                         # p: a placeholder whose loader holds layer
    gc.collect()
    assert key not in ops.DENSE_LAYERS                                   # dropped with its layer


def test_linear_checks_and_head_padding():
    gen = torch.Generator().manual_seed(1)
    bad = torch.nn.Module()
    m = Lin.EspLinearMethod("model.layers.0.self_attn.o_proj")
    m.create_weights(bad, 512, [256], 512, 256, torch.bfloat16)
    _load_linear(m, bad, [(None, 256)], gen, K=256)                      # input 256, the layer expects 512
    with pytest.raises(RuntimeError, match="do not fit"):
        m.process_weights_after_loading(bad)
    empty = torch.nn.Module()
    m.create_weights(empty, 256, [256], 256, 256, torch.bfloat16)
    with pytest.raises(RuntimeError, match="no trellis-coded"):
        m.process_weights_after_loading(empty)
    head = torch.nn.Module()
    h = Lin.EspLinearMethod("lm_head")
    h.create_weights(head, 256, [384], 256, 384, torch.bfloat16)
    h.process_weights_after_loading(head)                                # a drafter's head: nothing loaded, fine
    assert head.espalier.mats == [] and head.espalier.dense_key is None
    with pytest.raises(RuntimeError, match="never loaded"):
        h.apply(head, torch.zeros((1, 256)))
    padded = torch.nn.Module()
    h.create_weights(padded, 256, [512], 256, 512, torch.bfloat16)       # vocabulary padded past the matrix
    _load_linear(h, padded, [(None, 384)], gen)
    h.process_weights_after_loading(padded)
    assert padded.espalier.pad == 128 and ops.DENSE_LAYERS[padded.espalier.dense_key].n_out == 512


def _expert_weights(E, gen, D=256, I=128):
    for e in range(E):
        for proj, (k, n) in (("gate_proj", (D, I)), ("up_proj", (D, I)), ("down_proj", (I, D))):
            for suffix, t in WL.matrix_tensors(k, n, 2, "e2m1", gen).items():
                yield f"experts.{e}.{proj}.{suffix}", t


def test_moe_loader_and_checks():
    gen = torch.Generator().manual_seed(2)
    method = Moe.EspMoEMethod()
    assert method.topk_indices_dtype == torch.int32
    assert method.is_monolithic == Moe.ROUTE and method.mk_can_overlap_shared_experts == Moe.GROUPED
    layer = torch.nn.Module()
    layer.layer_name = "model.layers.0.mlp.experts"
    method.create_weights(layer, 3, 256, 128, torch.bfloat16)
    names = list(layer.load_weights(_expert_weights(3, gen)))
    assert names[:6] == ["w13_esp_trellis", "w13_suh", "w13_svh", "w13_mcg", "w13_esp_grid", "w13_esp_trellis"]
    assert "w2_esp_trellis" in names
    method.process_weights_after_loading(layer)
    assert len(layer.espalier.experts) == 3
    g, u, d = layer.espalier.experts[2]
    assert (g.in_features, g.out_features, d.in_features, d.out_features) == (256, 128, 128, 256)
    assert method.get_fused_moe_quant_config(layer) is None
    short = torch.nn.Module()
    method.create_weights(short, 4, 256, 128, torch.bfloat16)
    list(short.load_weights(_expert_weights(3, gen)))
    with pytest.raises(RuntimeError, match="missing"):
        method.process_weights_after_loading(short)
    odd = torch.nn.Module()
    method.create_weights(odd, 1, 256, 128, torch.bfloat16)
    with pytest.raises(ValueError, match="unexpected"):
        list(odd.load_weights([("experts.0.gate.esp_trellis", torch.zeros(1))]))
    with pytest.raises(ValueError, match="unknown suffix"):
        list(odd.load_weights([("experts.0.gate_proj.qweight", torch.zeros(1))]))
    gelu = torch.nn.Module()
    gelu.activation = "gelu"
    method.create_weights(gelu, 1, 256, 128, torch.bfloat16)
    list(gelu.load_weights(_expert_weights(1, gen)))
    with pytest.raises(NotImplementedError):
        method.process_weights_after_loading(gelu)


# ---- the plugin's patches, on stand-in vLLM classes
class _Quant:
    def __init__(self, name):
        self.name = name

    def get_name(self):
        return self.name


def test_salt_compute_hash(monkeypatch):
    class Cfg:
        def compute_hash(self):
            return "0123456789abcdef" * 2
    P.salt_compute_hash(Cfg)
    P.salt_compute_hash(Cfg)                                             # idempotent
    monkeypatch.setenv("ESPALIER_PREFILL_MODE", "tile")
    a = Cfg().compute_hash()
    monkeypatch.setenv("ESPALIER_PREFILL_MODE", "chunk")
    b = Cfg().compute_hash()
    monkeypatch.setenv("ESPALIER_PREFILL_MODE", "tile")
    assert a != b and len(a) == 32 and Cfg().compute_hash() == a


def test_patch_inductor():
    class Cfg:
        def __init__(self, quant):
            self.quant_config = quant
            self.compilation_config = types.SimpleNamespace(inductor_compile_config={})
            self.__post_init__()

        def __post_init__(self):
            self.compilation_config.inductor_compile_config["seen"] = True
    P.patch_inductor(Cfg)
    P.patch_inductor(Cfg)
    esp = Cfg(_Quant("espalier")).compilation_config.inductor_compile_config
    assert esp == {"seen": True, "benchmark_combo_kernel": False, "triton.autotune_at_compile_time": False}
    assert Cfg(_Quant("awq")).compilation_config.inductor_compile_config == {"seen": True}
    assert Cfg(None).compilation_config.inductor_compile_config == {"seen": True}


def _fake_mtp_module():
    m = types.ModuleType("fake_mtp")

    class Qwen3_5MultiTokenPredictor(torch.nn.Module):
        def __init__(self, *, vllm_config=None, prefix=""):
            super().__init__()
            self.embed_tokens = torch.nn.Embedding(10, 4)

    class Qwen3_5MTP(torch.nn.Module):
        def __init__(self, quant):
            super().__init__()
            self.quant_config = quant

        def load_weights(self, weights):
            return [n for n, _ in weights]
    m.Qwen3_5MultiTokenPredictor, m.Qwen3_5MTP = Qwen3_5MultiTokenPredictor, Qwen3_5MTP
    return m


def test_patch_mtp_module():
    m = _fake_mtp_module()
    P.patch_mtp_module(m)
    P.patch_mtp_module(m)
    vc = types.SimpleNamespace(quant_config=_Quant("espalier"))
    assert tuple(m.Qwen3_5MultiTokenPredictor(vllm_config=vc).embed_tokens.weight.shape) == (0, 4)
    other = types.SimpleNamespace(quant_config=_Quant("fp8"))
    assert tuple(m.Qwen3_5MultiTokenPredictor(vllm_config=other).embed_tokens.weight.shape) == (10, 4)
    names = [("model.lm_head.weight", 0), ("model.embed_tokens.weight", 0), ("model.layers.0.q.esp_trellis", 0)]
    assert m.Qwen3_5MTP(_Quant("espalier")).load_weights(iter(names)) == ["model.layers.0.q.esp_trellis"]
    assert len(m.Qwen3_5MTP(_Quant("fp8")).load_weights(iter(names))) == 3


def test_after_import(tmp_path, monkeypatch):
    name = "esp_after_import_probe_mod"
    (tmp_path / f"{name}.py").write_text("VALUE = 41\n")
    monkeypatch.syspath_prepend(str(tmp_path))
    seen = []
    P.after_import(name, lambda mod: seen.append(mod.VALUE + 1))
    assert seen == [] and name not in sys.modules                       # not imported by the hook itself
    __import__(name)
    assert seen == [42]
    P.after_import(name, lambda mod: seen.append(mod.VALUE))             # already imported: at once
    assert seen == [42, 41]
    del sys.modules[name]


def test_register_without_vllm():
    P.register()                                                         # the custom ops; no vLLM patches
    assert hasattr(torch.ops.espalier, "dense") and hasattr(torch.ops.espalier, "matmul")
    assert set(ops.PREFILL_MODES) == {"chunk", "gemm", "tile"}
