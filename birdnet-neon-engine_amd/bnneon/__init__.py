"""bnneon for MI355X: the host side of libbnneon_hip.

  hip       ctypes binding of the kernel-level C ABI (include/bnneon_hip.h)
  binding   the libbnneon host API (bnn_*) over libbnneon_hip.so
  pkgfmt    the .bnpk package format (writer and reader)
  s8pack    offline int8 weight quantization and packing
"""
