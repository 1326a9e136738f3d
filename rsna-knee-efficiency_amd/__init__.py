"""MI355X-native INT8 DenseNet169 encoder (gfx950 HIP kernels behind the reference's `Dense8SEncoder`
interface).  The directory name is not a Python identifier: load it as `rsna_knee_efficiency_amd` with
`load_package()` of `__graft_entry__.py` (tests/conftest.py and bench.py do).

Modules: `hip` (ctypes binding of libd8s_hip.so), `dense8s` (calibration, plan, tables, package,
runner), `densenet` (the float DenseNet169 the plan is built from), `build` (hipcc build).
"""
