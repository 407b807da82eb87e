"""MI355X (gfx950) paged-KV hot path with the module layout of the reference's
``engine`` package: ``engine.kernels.paged_attention`` (decode attention) and
``engine.runtime.paged_cache`` (KV pool, append, block copy). Put the directory that
holds this package (``inference-engine_amd/``) on ``sys.path`` to import it."""
