"""CPU oracle for the torchwarp alignment path -- TEST INFRASTRUCTURE ONLY.

Nothing in the shipped package (``torchwarp_amd``) imports this package. Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or as the timed CPU baseline),
never as the thing measured on the GPU.

It is a clean-room restatement, in plain PyTorch on CPU tensors, of the
reference's portable algorithms (paths relative to ``/root/reference``):

* ``udtw``   -- uDTW / soft-DTW dynamic program, analytic backward and the
  feature chain rule: ``src/torchwarp/udtw/_torch_dp.py:14-75``,
  ``src/torchwarp/udtw/_ops.py:149-154,179-183,200-211``,
  ``src/torchwarp/udtw/_autograd.py:24-29``,
  ``src/torchwarp/udtw/functional.py:62-91,104-209``.
* ``jeanie`` -- JEANIE 3-D DP over (viewpoints, t, u), its backward with an
  optional accumulator seed, FVM and the base costs:
  ``src/torchwarp/jeanie/_torch_dp.py:14-75``,
  ``src/torchwarp/jeanie/functional.py:28-175``,
  ``src/torchwarp/jeanie/fvm.py:15-67``,
  ``src/torchwarp/jeanie/distances.py:15-51``, ``src/torchwarp/sdtw.py:12-92``.
* ``paths``  -- hard (gamma = 0) DP with the backtrack order of
  ``src/torchwarp/paths.py:85-127``.
* ``brute``  -- brute-force enumeration of every monotone path (tiny sizes).
* ``udtw_tangent`` -- the second order of the uDTW DP (the derivative of the
  first-order gradient along a direction), what the reference's
  ``DPBackward.backward`` / ``jvp`` compute with torch.func over
  ``src/torchwarp/udtw/_autograd.py:32-74`` (``udtw/_ops.py:322-339``),
  written as explicit tangent recursions.
* ``udtw_ld`` -- the feature-path uDTW value and gradients in 80-bit
  extended precision, the judge of float64 rounding.

How each function is pinned (so that a dropped term, wrong sign, swapped
index or transposed operand fails a check) -- see ``tests/test_oracle.py``:

* the 147 float64 golden cases the reference ships
  (``tests/golden/reference.pt``, outputs of the official uDTW / JEANIE code),
  extracted as data into ``tests/golden/reference_cases.pt``;
* brute-force enumeration of all paths (value = softmin of path sums,
  gradient = path-probability matrix, hard argmin path);
* closed forms: 1x1 and 1xM grids, gamma -> 0 equals exact DTW, the
  normalize identity, K = 1 / shift 0 reduces JEANIE to soft-DTW;
* the analytic backward against autograd of the differentiable form;
* for ``udtw_tangent`` (``tests/test_oracle_tangent.py``): the reference's
  stored soft-DTW Hessian, double autograd through the differentiable form,
  finite differences of the analytic backward, Hessian symmetry.

Every function here is pinned by at least one of these; none is "parity
unpinned".
"""
