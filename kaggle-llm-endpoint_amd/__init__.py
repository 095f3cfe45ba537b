"""MI355X-native (gfx950) codebook-dequant MoE expert path: HIP kernels behind a C ABI (include/mi355moe.h),
loaded with ctypes, and the reference's ``ResidentFetch`` operator interface on top.

The directory name is not a Python identifier; it is imported as ``kaggle_llm_endpoint_amd`` through
``load_package()`` of ``__graft_entry__`` / ``tests/conftest.py``.
"""
from . import _lib, formats, gguf  # noqa: F401
from .resident import (Bf16Leaf, ExpertTable, ResidentFetch, bf16_leaf, bf16_mlp, bf16_project,  # noqa: F401
                       dequant, int8_mlp, int8_project, int8_project_many, int8_tile, matvec, mlp_partial,
                       moe_matvec, moe_decode, moe_prefill, moe_route, pack_planes_device, prefill_workspace_bytes,
                       ragged_plan, random_cb3_table, random_iq2s_table,
                       random_iq3s_table, random_iq4xs_table, random_kq_table, route, to_device_planes, tuning)

__all__ = ["Bf16Leaf", "ExpertTable", "ResidentFetch", "bf16_leaf", "bf16_mlp", "bf16_project", "dequant",
           "int8_mlp", "int8_project", "int8_project_many", "int8_tile",
           "matvec",
           "mlp_partial", "moe_matvec",
           "moe_decode",
           "moe_prefill", "moe_route", "pack_planes_device", "prefill_workspace_bytes", "ragged_plan", "route", "gguf", "random_cb3_table", "random_iq2s_table", "random_iq3s_table",
           "random_iq4xs_table", "random_kq_table", "to_device_planes", "tuning", "formats"]
