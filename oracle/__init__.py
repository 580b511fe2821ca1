"""CPU oracle for the OSCAR INT2 rotated KV-cache attention path.

TEST INFRASTRUCTURE ONLY.  This package is a NumPy restatement of the
reference's torch CPU path (``OSCAR_ASCEND_USE_TRITON=0``).  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker (or the timed CPU baseline).  The product
package ``oscar_amd`` never imports it and has no CPU fallback: its ops fail
loudly when the HIP library is missing.

Every function cites the reference file:line it restates.  How each function
is pinned (golden vectors / known-answer tests / closed forms / brute force)
is listed in ``PINNING`` below and exercised by ``tests/test_oracle_*.py``.

Modules
-------
fmt        INT2 slot contract: scales, quantize, pack, dequant, fp16 meta bytes.
store      rotation, sort-clip, scatter into packed caches, staging tags/window.
attention  streaming attention over INT2 history + current chunk, LSE merge.
backend    forward-level composition (write, window, read, inverse rotation,
           fresh-only prefill) on plain arrays.
cases      seeded generators for the BASELINE configurations.
"""

PINNING = {
    "fmt.pack/unpack": "exhaustive over all 256 byte values; hand-derived bytes (test_oracle_format)",
    "fmt.quantize": "floor(x+0.5) tie KAT, fp16-scale-before-coding KAT, float64 nearest-level "
                    "brute force, constant-vector KATs of tests/test_backend.py:139-146",
    "fmt.make_slot_bytes": "hand-derived 160-byte slot (scale/zero LE at 0..7, codes at 32/96)",
    "fmt.bf16_round": "bit-equal to torch's bfloat16 conversion incl. ties, subnormals, inf",
    "store.rotate": "bit-equal to exact rational dot products rounded once; R=I; Hadamard rows",
    "store.clip": "order-statistic KATs; tests/test_numeric.py:354-367 bound",
    "store.store_ref": "negative-slot no-op (tests/test_backend.py:56-75), split bytes == logical "
                       "slot (tests/test_numeric.py:82-103), last writer wins",
    "store.Staging": "reference lifecycle KATs: geometry, persist/recycle, collision + padding, "
                     "standalone invalidation; staging_order at the 2^24 boundary",
    "attention.attention_ref": "closed forms 3.0, 45/8, 75/9, -3, -4, all-ones of "
                               "tests/test_streaming_backend.py; float64 SDPA over independently "
                               "decoded history; empty rows; NaN propagation",
    "attention.merge_ref": "hand-derived edge cases (-inf parts, LSE +-1000, NaN); split-softmax identity",
    "attention.causal_prefill_ref": "float64 SDPA with GQA",
    "backend.forward": "fresh prefill == SDPA; rotated path == original-domain attention",
}
