"""MI355X-native decode-time linear layers of Breeze TTS 2.

Host-side mirror of the reference's modules (models/int4_linear.py,
models/fp8_linear.py, models/fused/) over the C ABI of libbzgemv.so
(include/bz_gemv.h).  Importing the package does not load the library;
the first GPU call does, and fails loudly if it was not built.
"""

__version__ = "0.1.0"
