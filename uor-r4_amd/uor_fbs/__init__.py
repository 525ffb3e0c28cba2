"""Host side of the MI355X SpiralCore/FBS decode path: seeded artifacts, the ctypes image of
include/uor_fbs.h, the UORLUT01 container reader and the binding of libuor_fbs_hip.so."""

from . import cabi, hip, synth, tables, uorlut  # noqa: F401
