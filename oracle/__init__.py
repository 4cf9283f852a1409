"""CPU oracle for the MatMulNBits / DynamicQuantizeLinear / MatMulInteger path.

Test infrastructure only (the parity checker).  Only tests/, the smoke() entry
point and bench.py's cpu_baseline leg may import it.
"""
