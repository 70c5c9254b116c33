"""Hash of the sources libcoda_mi355x.so is built from.

build.py compiles the hash into the library (coda_source_hash()); the loader
recomputes it from the sources beside the package and refuses a library
built from other sources, so a stale binary cannot stand in for changed
kernels.  No torch import: build.py uses this module too.
"""

from __future__ import annotations

import glob
import hashlib
import os
from typing import List, Optional

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC_DIR = os.path.join(os.path.dirname(PKG_DIR), "csrc")
INCLUDE_DIR = os.path.join(os.path.dirname(os.path.dirname(PKG_DIR)), "include")


def source_files() -> List[str]:
    """The kernel and ABI sources, the public header and the build script."""
    files = []
    for pat in ("*.hip", "*.h", "build.py"):
        files += glob.glob(os.path.join(CSRC_DIR, pat))
    files += glob.glob(os.path.join(INCLUDE_DIR, "*.h"))
    return sorted(files, key=os.path.basename)


def source_hash() -> Optional[str]:
    """16 hex digits of SHA-256 over (file name, contents) in name order, or
    None when the sources are not there (a library installed on its own)."""
    files = source_files()
    if not any(f.endswith(".hip") for f in files):
        return None
    h = hashlib.sha256()
    for f in files:
        h.update(os.path.basename(f).encode())
        h.update(b"\0")
        with open(f, "rb") as fh:
            h.update(fh.read())
        h.update(b"\0")
    return h.hexdigest()[:16]
