"""qw3_amd: the MI355X (gfx950) backend for DS5's GQA attention path.

    qw3_amd.build.build()  compiles qw3_amd/csrc/*.hip into qw3_amd/libds5hip.so
    qw3_amd.hip            the DS5 Ctx / kernel-provider interface over that library

The C ABI is declared in include/ds5_hip.h.
"""

__all__ = ["hip", "build"]
