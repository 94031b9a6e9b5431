"""vllm_espalier on MI355X (gfx950): the plugin's Python surface over hand-written HIP kernels.

Registered with vLLM through the vllm.general_plugins entry point (register()); the kernels live in
libespalier_hip.so (C ABI: include/espalier.h) and are reached through the espalier_ext torch extension.

register() (vllm_espalier/__init__.py:105-112) imports the quantisation config (which registers quant_method
"espalier" with vLLM) and the custom ops, and adjusts three things of vLLM's, each written against the class or module
it is given so it can be checked without vLLM:
  * salt_compute_hash: the ESPALIER_* switches change which custom ops a compiled graph calls but are not vLLM
    config, so they are mixed into VllmConfig.compute_hash, the key of vLLM's compile cache (:12-22);
  * patch_inductor: for Espalier checkpoints, inductor's combo-kernel benchmarking and compile-time Triton autotuning
    are turned off (both run on random copies of a kernel's inputs, which for the bf16 embedding is a ~1 GB
    transient) (:83-101);
  * patch_mtp_module: an MTP drafter of an Espalier checkpoint drops its own embedding right after construction and
    skips loading its own head and embedding, which vLLM replaces with the target's anyway (:25-80); applied when
    vLLM's qwen3_5_mtp module is imported (after_import), never importing it early.
"""
import hashlib
import os
import sys

# the switches that change which custom ops a compiled graph calls (vllm_espalier/__init__.py:12)
SWITCHES = ("ESPALIER_FUSED_DENSE", "ESPALIER_GROUPED_EXPERTS", "ESPALIER_FUSED_ROUTING", "ESPALIER_PREFILL_MODE")
MTP_MODULE = "vllm.model_executor.models.qwen3_5_mtp"


def switches_salt() -> str:
    """The switch settings, as mixed into vLLM's compile-cache hash."""
    return ",".join(f"{k}={os.environ.get(k, '')}" for k in SWITCHES)


def _espalier_quant(cfg) -> bool:
    from .config import NAME
    return cfg is not None and cfg.get_name() == NAME


def salt_compute_hash(cls) -> None:
    """cls.compute_hash(...) -> the same-length hex digest of (its hash, the switch settings). Idempotent."""
    inner = cls.compute_hash
    if getattr(inner, "_esp", False):
        return

    def compute_hash(self, *args, **kwargs):
        h = inner(self, *args, **kwargs)
        return hashlib.sha256(f"{h}|{switches_salt()}".encode()).hexdigest()[:len(h)]
    compute_hash._esp = True
    cls.compute_hash = compute_hash


def patch_inductor(cls) -> None:
    """After cls.__post_init__, an Espalier config's inductor settings skip benchmarking on input copies. Idempotent."""
    inner = cls.__post_init__
    if getattr(inner, "_esp", False):
        return

    def post_init(self, *args, **kwargs):
        inner(self, *args, **kwargs)
        if _espalier_quant(getattr(self, "quant_config", None)):
            opts = self.compilation_config.inductor_compile_config
            opts["benchmark_combo_kernel"] = False
            opts["triton.autotune_at_compile_time"] = False
    post_init._esp = True
    cls.__post_init__ = post_init


def patch_mtp_module(m) -> None:
    """The drafter classes of vLLM's qwen3_5_mtp module: for an Espalier checkpoint the predictor's embedding is
    emptied after construction, and the drafter's loader skips lm_head and embed_tokens tensors. Idempotent."""
    import torch
    pred, mtp = m.Qwen3_5MultiTokenPredictor, m.Qwen3_5MTP
    if getattr(pred.__init__, "_esp", False):
        return
    init0, load0 = pred.__init__, mtp.load_weights

    def init(self, *args, **kwargs):
        init0(self, *args, **kwargs)
        vc = kwargs.get("vllm_config")
        if vc is not None and _espalier_quant(vc.quant_config) and hasattr(self, "embed_tokens"):
            w = self.embed_tokens.weight
            self.embed_tokens.weight = torch.nn.Parameter(w.new_empty((0, w.shape[1])), requires_grad=False)

    def load_weights(self, weights):
        if _espalier_quant(getattr(self, "quant_config", None)):
            weights = ((n, w) for n, w in weights if "lm_head" not in n and "embed_tokens" not in n)
        return load0(self, weights)

    init._esp = True
    pred.__init__ = init
    mtp.load_weights = load_weights


def after_import(name: str, fn) -> None:
    """fn(module) once module `name` has been imported (now, if it already is), without importing it: importing a
    vLLM model module initialises the GPU runtime, which the API process must not do."""
    if name in sys.modules:
        fn(sys.modules[name])
        return
    import importlib.abc
    import importlib.util

    class _Hook(importlib.abc.MetaPathFinder):
        def find_spec(self, fullname, path, target=None):
            if fullname != name:
                return None
            sys.meta_path.remove(self)
            spec = importlib.util.find_spec(fullname)
            if spec is None or spec.loader is None:
                return spec
            run = spec.loader.exec_module

            def exec_module(module):
                run(module)
                fn(module)
            spec.loader.exec_module = exec_module
            return spec

    sys.meta_path.insert(0, _Hook())


def register():
    """vLLM plugin entry point."""
    from . import config, ops  # noqa: F401  (quant_method "espalier" and the espalier::* ops)
    if not config.HAVE_VLLM:
        return
    from vllm.config import VllmConfig
    salt_compute_hash(VllmConfig)
    patch_inductor(VllmConfig)
    after_import(MTP_MODULE, patch_mtp_module)
