"""Loads the product package from its directory (its name, llama.rs_amd, is
not a Python identifier, so it is loaded by path as module `llama_rs_amd`)."""
import importlib.util
import os
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_product():
    if "llama_rs_amd" in sys.modules:
        return sys.modules["llama_rs_amd"]
    pkg_dir = os.path.join(REPO, "llama.rs_amd")
    spec = importlib.util.spec_from_file_location(
        "llama_rs_amd", os.path.join(pkg_dir, "__init__.py"),
        submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["llama_rs_amd"] = mod
    spec.loader.exec_module(mod)
    return mod
