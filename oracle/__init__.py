"""CPU oracle for the ERNIE 5.5 attention KV-cache hot path.

TEST INFRASTRUCTURE ONLY. This package restates, in numpy (with torch on the
CPU only where a library routine pins a result), the arithmetic of the
reference plugin's KV-cache path:

* ``fp8``       -- OCP e4m3fn codec and the UE8M0 per-token scale rule;
* ``paged``     -- slot math and the paged page layouts (latent and indexer K);
* ``hca``       -- HCA append, 128->1 span compressor and the window ring;
* ``indexer``   -- indexer prep (Hadamard, NeoX partial RoPE, q quant),
                   lightning-indexer scoring and exact top-k;
* ``merge``     -- ``merge_swa_topk`` and logical->global index conversion;
* ``decode``    -- sparse MLA decode with an attention sink.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker: the product path (the HIP
library under ``vllm-ernie_amd``) never calls into it and raises when the
compiled library is missing.

Reference citations are ``path:line`` into the baidu/vLLM-ERNIE tree
(``src/vllm_ernie/models/ernie5_5/...``).  Parts of the path whose arithmetic
lives in vLLM 0.32.0 (absent here) are restated from their call sites and are
marked "parity unpinned" where no reference test or closed form fixes them.
"""
