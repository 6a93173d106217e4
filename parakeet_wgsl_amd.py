"""Import shim for the package directory `parakeet.wgsl_amd/`.

A dotted directory name is not importable as a Python package, so this module
loads that directory as the package `parakeet_wgsl_amd`; afterwards
`import parakeet_wgsl_amd.palette_abi` and friends resolve inside it.
"""
import importlib.util
import os
import sys

_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "parakeet.wgsl_amd")
_spec = importlib.util.spec_from_file_location(
    __name__, os.path.join(_DIR, "__init__.py"), submodule_search_locations=[_DIR])
_module = importlib.util.module_from_spec(_spec)
sys.modules[__name__] = _module
_spec.loader.exec_module(_module)
