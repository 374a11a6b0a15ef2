"""CPU oracle for the HilbertA inference attention path -- TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The shipped package ``hilberta_amd`` never imports anything here and
fails loudly when its HIP library is missing.

Modules
-------
topology     numpy restatement of geometry.py / plan.py / bridge_k.py /
             paired_metadata.py / sparse_kernel.validate_metadata (block tables).
mask_oracle  an independent second algorithm for the same tables, restated from
             the reference's ordering-independent tests/topology_oracle.py
             (rolled-sequence coordinates, token-level counting).
attention    fp32 dense masked attention + per-row logsumexp with the reference's
             mask semantics (sparse_kernel.explicit_mask, mask_reference.joint_mask).

Pinning (see each module's header): known answers from the reference's tests
(test_plan.py:54-59, test_paired_metadata.py:46-55), the reference's own data
file website/data/demo.json, the second algorithm in mask_oracle, closed forms
(Hilbert locality, permutation properties), brute force on tiny inputs, and
library routines (torch SDPA / logsumexp) for the attention.
"""
