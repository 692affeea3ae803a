"""CPU oracle of NamiTorch's optimizer-step path — TEST INFRASTRUCTURE ONLY.

A NumPy restatement of the reference's CPU (NumPy backend) algorithms,
operation for operation, used to check the MI355X kernels:

* ``oracle.adam``  — Adam/AdamW update (optim/adam.py:27-42, 69-94;
  optim/_common.py:39-73), plus the master-weight / bfloat16 extensions;
* ``oracle.clip``  — _total_norm and clip_grad_norm_ (optim/clip_grad.py:63-112);
* ``oracle.scaler`` — GradScaler unscale_/_finite/update (amp.py:114-234);
* ``oracle.lowp``  — bfloat16 emulation (RNE) on uint16 bit patterns;
* ``oracle.grads`` — gradient accumulation (autograd.py:198-205).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed
CPU baseline; the product (``namitorch_amd``) never imports it.

How each function is pinned (checked independently of this restatement) is
listed in its docstring; tests/test_oracle.py runs those checks.
"""
