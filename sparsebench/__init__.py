"""The reference's import path for this build's MoE forward path.

Callers of saransh-debugs/SparseBench write `from sparsebench import _C`,
`sparsebench.moe.moe_forward`, `sparsebench.routing.route_device` and
`sparsebench.spmm.sdd` / `dsd` (sparsebench/__init__.py:1-5,
setup.py:14, csrc/bindings.cpp:5). Each of those names is the module of
`sparsebench_amd` that implements it on gfx950, registered under this
package: `sparsebench.moe is sparsebench_amd.moe`, so there is one copy of
every module and patching one name patches both.

Only the forward path's modules are registered (_MODULES). The reference's
benchmark and test support modules (sparsebench.reference, .timing,
.baselines) and the CPU functions of its sparsebench.topology
(build_topology, bsr_to_dense, dense_to_bsr) are not part of this build and
raise ImportError / AttributeError here.

Importing this package does not load the HIP library; that happens on the
first op call, as in `sparsebench_amd`.
"""

import importlib
import sys

_MODULES = ("_C", "moe", "routing", "spmm", "topology", "token_rounding", "workloads")

for _name in _MODULES:
    _module = importlib.import_module(f"sparsebench_amd.{_name}")
    sys.modules[f"{__name__}.{_name}"] = _module
    globals()[_name] = _module

del _name, _module
