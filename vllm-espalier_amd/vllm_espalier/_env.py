"""Environment switches (ESPALIER_*), read as the reference reads them (vllm_espalier/_env.py:5-6)."""
import os


def env(name: str, default: str | None = None) -> str | None:
    return os.environ.get(name, default)
