"""Locations of the in-tree native build outputs."""
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_DIR = os.path.join(PKG_DIR, "lib")
BIN_DIR = os.path.join(PKG_DIR, "bin")
INCLUDE_DIR = os.path.join(REPO_DIR, "include")


def hip_lib() -> str:
    return os.path.join(LIB_DIR, "libstrasgpt_hip.so")


def synth_exe() -> str:
    path = os.path.join(BIN_DIR, "strasgpt-synth")
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run __graft_entry__.build()")
    return path


def driver_exe() -> str:
    return os.path.join(BIN_DIR, "strasgpt")
