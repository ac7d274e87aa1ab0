"""CPU oracle for the run-time SDM mixer (RunTimeSdm) -- TEST INFRASTRUCTURE ONLY.

Nothing in the product package imports this package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and there only to check results (or, for ``cpu_baseline``, as the
timed CPU restatement), never as a path that produces product results.

Modules
-------
``sdm_fp64``   numpy float64 restatement: product-key addressing (and a brute-force full-grid search), softmax /
               gate / RMSNorm / out-norm in closed form, and the token-by-token recurrence of the memory.
``sdm_torch32`` torch float32 CPU restatement that follows the reference's op sequence (F.normalize, einsum, topk,
               dense chunk scatter and matmuls), so its addressing bits equal the reference's when run with the same
               torch build.  It is also the timed CPU baseline.
``sdm_grad64`` float64 torch restatement of the core (and of TrainedSdm's table read) for fixed picks, differentiated
               by torch autograd: the oracle of the backward kernels.

Pinning (what each oracle function is checked against in ``tests/``):
  * ``sdm_torch32.pk_address`` -- bit-exact against golden vectors written by the reference's own ``pk_address``
    (``tests/golden/pk_address_*.npz``), including exact-tie cases.
  * ``sdm_fp64.pk_address`` -- equals ``sdm_fp64.pk_address_bruteforce`` (full n_sub^2 grid) on every input, and the
    golden ids wherever the fp64 margin between the k-th and (k+1)-th score exceeds 1e-6.
  * ``sdm_fp64.scan_recurrence`` -- closed forms: previous-token head (fade 0), never-fading head (fade 1, a plain
    prefix sum), gate ~ 0 gives a zero read, and equality with ``sdm_torch32`` chunked form for chunk sizes
    1, 5, 7, 23, 64, 128 and T.
  * softmax / sigmoid / RMSNorm / out-norm -- textbook closed forms, checked on hand-computed values.
  * ``sdm_grad64.core_from_picks`` / ``table_from_picks`` -- forward equal to ``sdm_fp64`` (token recurrence, table
    read) to 1e-12; every autograd gradient equal to central finite differences of the ``sdm_fp64`` forward (picks
    recomputed and checked not to move); the fade identity lam dL/dlam = sum_t t P_t - sum_s (s+1) Q_s.
"""
