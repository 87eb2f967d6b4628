"""folder_paths stand-in: files live under ROOTS[kind]."""
import os

ROOTS: dict = {}


def get_filename_list(kind):
    d = ROOTS.get(kind)
    return sorted(os.listdir(d)) if d and os.path.isdir(d) else []


def get_full_path(kind, name):
    d = ROOTS.get(kind)
    p = os.path.join(d, name) if d else None
    return p if p and os.path.exists(p) else None


def get_full_path_or_raise(kind, name):
    p = get_full_path(kind, name)
    if p is None:
        raise FileNotFoundError(name)
    return p
