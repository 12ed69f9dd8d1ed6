"""CPU oracle for mlx-hip parity tests (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` use this package, and only as the checker / the timed CPU
baseline. The mlx-hip library and its Python package never import it.
"""
