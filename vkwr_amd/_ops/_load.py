"""Loads a native extension module of vkwr_amd, failing loudly if it is absent."""
import importlib


def load_ext(name):
    try:
        return importlib.import_module(f"vkwr_amd.{name}")
    except ImportError as e:  # pragma: no cover - exercised only on a broken install
        raise ImportError(
            f"vkwr_amd native extension '{name}' is not built or cannot be loaded ({e}). "
            "Build it with `python vkwr_amd/_build.py` (gfx950 HIP kernels); "
            "there is no CPU fallback."
        ) from e
