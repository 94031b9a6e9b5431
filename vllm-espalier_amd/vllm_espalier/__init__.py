"""vllm_espalier on MI355X (gfx950): the plugin's Python surface over hand-written HIP kernels.

Registered with vLLM through the vllm.general_plugins entry point (register()); the kernels live in
libespalier_hip.so (C ABI: include/espalier.h) and are reached through the espalier_ext torch extension.

register() (the plugin entry of the reference's vllm_espalier/__init__.py:105-112) imports the quantisation config
(which registers quant_method "espalier" with vLLM) and the custom ops, then adjusts three things of vLLM's. Each
adjustment is a function of the class or module it is given, so it can be checked without vLLM, and each is applied
at most once (wrap_method marks what it has wrapped):
  * salt_compute_hash: VllmConfig.compute_hash keys vLLM's compile cache, but the ESPALIER_* switches, which change
    which custom ops a compiled graph calls, are not vLLM config; their settings are mixed into the hash;
  * patch_inductor: for Espalier checkpoints, inductor's combo-kernel benchmarking and compile-time Triton autotuning
    are turned off; both run kernels on random copies of their inputs, a ~1 GB transient for the bf16 embedding;
  * patch_mtp_module: vLLM gives an MTP drafter the target's embedding and LM head, but only after the drafter has
    built its own embedding and loaded its own head. For an Espalier checkpoint the drafter's embedding is released
    right after construction and its loader skips both. The module is patched when vLLM imports it
    (after_import), never imported early: importing a vLLM model module initialises the GPU runtime, which vLLM's
    API process must not do.
"""
import hashlib
import os
import sys

# the switches that change which custom ops a compiled graph calls
SWITCHES = ("ESPALIER_FUSED_DENSE", "ESPALIER_GROUPED_EXPERTS", "ESPALIER_FUSED_ROUTING", "ESPALIER_PREFILL_MODE")
MTP_MODULE = "vllm.model_executor.models.qwen3_5_mtp"
# inductor settings an Espalier checkpoint switches off
INDUCTOR_OFF = ("benchmark_combo_kernel", "triton.autotune_at_compile_time")
# checkpoint names an MTP drafter of an Espalier checkpoint does not load (vLLM installs the target's)
DRAFTER_SKIPS = ("lm_head", "embed_tokens")
_MARK = "_espalier_wrapped"


def switches_salt() -> str:
    """The switch settings, as mixed into vLLM's compile-cache hash."""
    return ",".join(f"{k}={os.environ.get(k, '')}" for k in SWITCHES)


def espalier_quant(quant_config) -> bool:
    """Whether a vLLM quantisation config (or None) is this plugin's."""
    from .config import NAME
    return quant_config is not None and quant_config.get_name() == NAME


def wrap_method(cls, name: str, make) -> None:
    """cls.name = make(the current cls.name), unless cls.name is already a wrapper made here."""
    current = getattr(cls, name)
    if getattr(current, _MARK, False):
        return
    wrapper = make(current)
    setattr(wrapper, _MARK, True)
    setattr(cls, name, wrapper)


def salt_compute_hash(cls) -> None:
    """cls.compute_hash(...) -> a digest of (its own hash, the switch settings), as long as its own hash."""
    def make(compute_hash):
        def salted(self, *args, **kwargs):
            own = compute_hash(self, *args, **kwargs)
            digest = hashlib.sha256(own.encode())
            digest.update(b"|espalier|" + switches_salt().encode())
            return digest.hexdigest()[:len(own)]
        return salted
    wrap_method(cls, "compute_hash", make)


def patch_inductor(cls) -> None:
    """After cls.__post_init__, an Espalier config's inductor settings run no benchmarks on input copies."""
    def make(post_init):
        def post_init_espalier(self, *args, **kwargs):
            post_init(self, *args, **kwargs)
            if espalier_quant(getattr(self, "quant_config", None)):
                self.compilation_config.inductor_compile_config.update(dict.fromkeys(INDUCTOR_OFF, False))
        return post_init_espalier
    wrap_method(cls, "__post_init__", make)


def _release_embedding(module) -> None:
    """Replace module.embed_tokens' weight by an empty [0, hidden] parameter of its dtype and device."""
    import torch
    w = module.embed_tokens.weight
    empty = torch.empty((0, w.shape[1]), dtype=w.dtype, device=w.device)
    module.embed_tokens.weight = torch.nn.Parameter(empty, requires_grad=False)


def patch_mtp_module(module) -> None:
    """The drafter classes of vLLM's qwen3_5_mtp module, for an Espalier checkpoint: the predictor's embedding is
    released after construction, and the drafter's loader skips the DRAFTER_SKIPS tensors."""
    def make_init(init):
        def init_espalier(self, *args, **kwargs):
            init(self, *args, **kwargs)
            config = kwargs.get("vllm_config")
            if config is not None and espalier_quant(config.quant_config) and hasattr(self, "embed_tokens"):
                _release_embedding(self)
        return init_espalier

    def make_load(load_weights):
        def load_espalier(self, weights):
            if espalier_quant(getattr(self, "quant_config", None)):
                weights = (item for item in weights if not any(part in item[0] for part in DRAFTER_SKIPS))
            return load_weights(self, weights)
        return load_espalier

    wrap_method(module.Qwen3_5MultiTokenPredictor, "__init__", make_init)
    wrap_method(module.Qwen3_5MTP, "load_weights", make_load)


class _AfterImport:
    """A meta-path finder that runs callbacks on a module right after its first import. For a module with pending
    callbacks it finds the spec through the rest of sys.meta_path and returns it with its loader wrapped, so the
    callbacks run once the module has executed; it stays installed while any callback is pending."""

    def __init__(self):
        self.pending: dict[str, list] = {}

    def find_spec(self, fullname, path=None, target=None):
        callbacks = self.pending.pop(fullname, None)
        if callbacks is None:
            return None
        if not self.pending:
            sys.meta_path.remove(self)
        import importlib.util
        spec = importlib.util.find_spec(fullname)
        if spec is None or spec.loader is None:
            return spec
        spec.loader = _CallbackLoader(spec.loader, callbacks)
        return spec


class _CallbackLoader:
    """Delegates to a module's own loader, then calls the callbacks with the executed module."""

    def __init__(self, loader, callbacks):
        self.loader, self.callbacks = loader, callbacks

    def create_module(self, spec):
        return self.loader.create_module(spec)

    def exec_module(self, module):
        self.loader.exec_module(module)
        for fn in self.callbacks:
            fn(module)

    def __getattr__(self, name):
        return getattr(self.loader, name)


_AFTER_IMPORT = _AfterImport()


def after_import(name: str, fn) -> None:
    """fn(module) once module `name` is imported (at once if it already is), without importing it."""
    if name in sys.modules:
        fn(sys.modules[name])
        return
    _AFTER_IMPORT.pending.setdefault(name, []).append(fn)
    if _AFTER_IMPORT not in sys.meta_path:
        sys.meta_path.insert(0, _AFTER_IMPORT)


def register():
    """vLLM plugin entry point."""
    from . import config, ops  # noqa: F401  (quant_method "espalier" and the espalier::* ops)
    if not config.HAVE_VLLM:
        return
    from vllm.config import VllmConfig
    salt_compute_hash(VllmConfig)
    patch_inductor(VllmConfig)
    after_import(MTP_MODULE, patch_mtp_module)
