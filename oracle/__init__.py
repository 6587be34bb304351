"""CPU oracle for the FP8-V decode hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports, links or calls this
package; only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker (or, for ``cpu_baseline``, as the timed CPU
restatement of the reference path).

Contents (each function cites the reference file:line it restates):

* ``oracle.fp8``       -- from-spec OCP E4M3FN codec (C, ``fp8_e4m3.c``) behind ctypes.
* ``oracle.quant``     -- ``quantize_kv_fp8`` / ``dequantize_kv_fp8`` restated in torch-CPU
                          (specdec/engine/model_self.py:300-320), with both scale-division
                          semantics (CPU true division, CUDA/ROCm reciprocal multiply).
* ``oracle.attention`` -- the eager GQA attention core (model_self.py:294-298, 739-776;
                          specdec/kernels/reference.py:33-70), an fp64 ground truth and the
                          full v_fp8 read/append step (model_self.py:689-728, 778-800).
* ``oracle.paged``     -- numpy restatement of the paged cache layout this build uses
                          (write by slot mapping, gather back to contiguous (B,KV,T,D)).

Pinning (what checks each function independently of its own formula) is listed in
each module's docstring.  Functions with no independent check say "parity unpinned".
"""
