"""MI355X (gfx950) paged-attention path of a paged-KV LLM server.

The operator API mirrors the reference server's (app/model, app/memory,
app/scheduler): PagedStepContext, paged_attention_forward, AttentionBackend /
select_backend and PagedKVCacheManager.  Behind it, HIP kernels in
``libpaged_attention_amd.so`` (C ABI: include/paged_attention_amd.h) pack the
ragged batch, write K/V into the paged cache, and run split-K decode and
MFMA chunked-prefill attention.  Import submodules explicitly, e.g.
``importlib.import_module(PACKAGE + ".paged_ops")``.
"""

PACKAGE_NAME = __name__
