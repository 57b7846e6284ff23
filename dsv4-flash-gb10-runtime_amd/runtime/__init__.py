"""Host side of the MI355X decode kernels: ctypes bindings with the reference's
binding contract (runtime/*_binding.py), the seeded input generator, and the
routed-MoE layer driver. Each binding loads its kernel library from
``../kernel/<dir>/lib*.so`` (the reference's relative layout) unless the
reference's ``*_LIB`` environment variable names another path.
"""
