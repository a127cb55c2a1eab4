"""Import-for-side-effect module that registers every built-in plugin
(the role of src/teamredbench/builtin.py)."""
from teamredbench_amd.benchmarks import hbm, mfu  # noqa: F401
from teamredbench_amd.metrics import common  # noqa: F401
from teamredbench_amd.native import builtin as native_builtin  # noqa: F401
from teamredbench_amd.profiling import builtin as profiling_builtin  # noqa: F401
