"""ORACLE — test infrastructure only.

A CPU restatement of the reference's per-token forward path
(miracle_reasoning/model.py, kernels.cl, config.py).  It exists to check the HIP
library and to time a CPU baseline.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker; the shipped package never imports, links or calls anything here.

Layout:
  kernels.c / kernels.py   the 13 reference kernels, same per-work-item arithmetic
  config.py                geometry, RoPE tables and the weight-shape table
  model.py                 per-family orchestration of one token step, prefill,
                           decode and generate
  device.py                the reference backend's method surface over the C
                           kernels (used only to write golden fixtures)

Parity pinning (which check pins which function) is listed in each module's
docstring.
"""
