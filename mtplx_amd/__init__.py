"""mtplx_amd — MI355X-native speculative-verify hot path of MTPLX.

Python call surface of the reference's verify path (``verify_qmv``,
``nax_verify``, ``verify_kernels``, ``ragged_kv_cache``, ``ragged_attention``,
``moe_sorted_gather``, ``sampling``/``fast_sampling``/``speculative``) over hand-written gfx950
HIP kernels reached through the C ABI in ``include/mtplx_amd.h``.
"""

__version__ = "0.1.0"
