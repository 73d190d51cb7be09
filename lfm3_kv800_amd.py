"""Import shim: `import lfm3_kv800_amd` loads the package that lives in the directory lfm3-kv800_amd/ (a directory
name Python cannot import directly). The shim replaces itself in sys.modules with that package."""
import importlib.util as _util
import os as _os
import sys as _sys

_ROOT = _os.path.join(_os.path.dirname(_os.path.abspath(__file__)), "lfm3-kv800_amd")
_spec = _util.spec_from_file_location(__name__, _os.path.join(_ROOT, "__init__.py"), submodule_search_locations=[_ROOT])
_mod = _util.module_from_spec(_spec)
_sys.modules[__name__] = _mod
_spec.loader.exec_module(_mod)
