"""HIP kernels of the verify path behind the reference's kernel-module API (slotstream_spark/kernels)."""
