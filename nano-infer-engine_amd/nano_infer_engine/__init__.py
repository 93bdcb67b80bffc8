"""nano_infer_engine for MI355X: the paged-attention path on hand-written gfx950 kernels.

Modules mirror the reference engine's layout (``block_allocator``,
``paged_cache``, ``layers``, ``models``, ``generation``); ``_native`` binds
the HIP library and ``paged_batch`` builds the per-forward device metadata.
"""

__version__ = "0.1.0"
