"""MI355X-native int4 MatMulNBits / int8 DynamicQuantizeLinear -> MatMulInteger.

The compute path is libmmnb.so (hand-written HIP for gfx950 behind a C ABI,
declared in include/mmnb.h).  ``ops`` mirrors the reference's Dart operator
functions over that ABI.
"""
