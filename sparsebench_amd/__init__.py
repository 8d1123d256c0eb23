"""MI355X-native MegaBlocks-style MoE forward path (routing -> SDD+GELU -> DSD -> combine).

A drop-in for the reference's sparsebench package on this path:
`sparsebench_amd.moe.moe_forward`, `sparsebench_amd.routing.route_device`,
`sparsebench_amd.spmm.sdd` / `dsd` and `sparsebench_amd._C` keep the
reference's names, arguments and results. The compute runs in hand-written
gfx950 HIP kernels of libsparsebench_hip.so, called through its C ABI.

The HIP library is loaded lazily (first op call), so the pure-Python parts
import on machines without a GPU.
"""
