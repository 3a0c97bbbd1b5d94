"""Synaptik MI355X (gfx950) execution backend: HIP kernels behind a C ABI (libsynaptik_hip.so),
with a host-side mirror of the reference's backend SPI and training surface."""
from .native import HipContext, HipBuffer, HipProgram, load_library  # noqa: F401
