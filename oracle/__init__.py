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
    "fmt.vector_scales": "closed form (fp16 RNE of min/max, 2^-14 floor); constant-vector KAT",
    "fmt.quantize": "brute force vs exhaustive threshold table; floor(x+0.5) tie KAT",
    "fmt.pack/unpack": "exhaustive over all 256 byte values",
    "fmt.make_slot_bytes": "byte positions KAT (scale/zero LE at 0..7, codes at 32/96)",
    "store.rotate": "R=I exactness; Hadamard closed form vs fp64; order independence",
    "store.clip": "k-th order statistic KAT",
    "store.store_ref": "negative-slot no-op, last-writer-wins KATs, R=I round trip",
    "store.staging_write_ref": "reference lifecycle KATs (persist, recycle, collision, padding)",
    "attention.attention_ref": "fp64 brute-force softmax; closed forms 3.0, 45/8, 75/9, -3, -4",
    "attention.merge_ref": "edge cases: -inf parts, LSE +-1000, NaN propagation",
    "backend.forward_ref": "SDPA equality without history; rotation invariance",
}
