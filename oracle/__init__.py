"""CPU oracle for the DSQG offset-gather path -- TEST INFRASTRUCTURE ONLY.

Restatements of the reference's mathematics used to check the HIP library:
only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the timed CPU baseline.
The product (dwarf-v2_amd/) never imports it and has no CPU fallback.

  dsqg_ref  kernels/dsqg_attention_v22.py:2560-2688 (eager oracle), with the
            GPU path's conventions (dsqg:760-763, 845-851, 2265-2268)
  ema_ref   kernels/causal_ema_scan.py:3-11, 511-538
  q6_ref    the q6 cache format (no reference counterpart)
  probe_ref phase-probe features, dsqg:275-369 (kernels), 422-451 (eager)
  npci_ref  NPCI kv_inject rotation, dsqg:221-254 (called at 3213-3224)
"""
