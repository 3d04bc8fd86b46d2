"""Locations of the in-tree built libraries."""
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG_DIR, "_lib")


def lib_path(name: str) -> str:
    return os.path.join(LIB_DIR, name)
