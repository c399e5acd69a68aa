"""The oracle: CPU restatements of the reference's selective-scan path.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py`` may import, call, link or execute anything
under ``oracle/``, and only as the checker.  The product package
(``mlx_vision_mamba_amd``) never imports it.

* ``scan_oracle``  float64 numpy restatement (forward, VJP, chunked,
                   two-pass, direction remaps).
* ``ref_lib``      ctypes binding of ``scan_ref.c`` (float64 C restatement,
                   built by ``oracle/Makefile``).
* ``torch_ref``    torch restatements: the reference's ``sequential`` and
                   ``chunked`` scan modes with autograd (the CPU baseline) and
                   a functional float64 MambaBlock / direction block /
                   VisionMamba used for module parity.

Pinning status of every function is listed in ``scan_oracle``'s header and in
tests/test_oracle.py.
"""
