"""CPU oracle for the Flash-DMLA kernels (test infrastructure only; see dmla_ref.py)."""
