"""Locations inside the repository."""

import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
SRC_ROOT = os.path.dirname(PKG_DIR)          # voyager-compiler-2_amd/
REPO_ROOT = os.path.dirname(SRC_ROOT)
CSRC_DIR = os.path.join(SRC_ROOT, "csrc")
INCLUDE_DIR = os.path.join(REPO_ROOT, "include")
