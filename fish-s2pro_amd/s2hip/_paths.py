"""Locations of the in-tree native libraries."""

import os

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT_DIR = os.path.dirname(PACKAGE_DIR)  # fish-s2pro_amd/
CSRC_DIR = os.path.join(ROOT_DIR, "csrc")
REPO_DIR = os.path.dirname(ROOT_DIR)
INCLUDE_DIR = os.path.join(REPO_DIR, "include")


def hip_library() -> str:
    return os.path.join(PACKAGE_DIR, "libs2hip.so")


def synth_library() -> str:
    return os.path.join(PACKAGE_DIR, "libs2synth.so")
