"""CPU oracle of the int8 path -- TEST INFRASTRUCTURE ONLY.

q8ref.c / q8ref.h   plain C restatement of the reference arithmetic
q8ref.py            numpy front end (ctypes)
q8ref.js            JavaScript mirror of the reference's generated CPU kernels
configs.py          expected outputs of the five workloads
Only tests/, __graft_entry__.smoke() (as the checker) and bench.py's
cpu_baseline leg may use this package.
"""
