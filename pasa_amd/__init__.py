"""pasa_amd: the PISA-PG sparse-attention hot path of PASA, native to MI355X (gfx950).

Kernels live in libpasa_amd.so (C ABI, include/pasa.h), built in-tree by
``python -m pasa_amd.build``.  Import surface:

* ``pasa_amd.ops``        pisa_pg_attention and its stages (block_stats, select_blocks, sparse_attn)
* ``pasa_amd.placement``  frame-major <-> token-major permutation
* ``pasa_amd.processors`` Wan / HunyuanVideo attention processors and installers
* ``pasa_amd.density``    per-timestep density tables
"""
__version__ = "0.1.0"
