"""File names of the package's native libraries (shared by the loader and the build)."""

import os
import sysconfig

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libfqkv_decode.so"
# the same library built with per-stage clock stamps in the decode kernel (diagnostics only)
TIMELINE_LIB_NAME = "libfqkv_decode_timeline.so"
EXT_NAME = "_fqkv_torch"


def ext_filename():
    return EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX")
