"""Verified reads of map files: the load-time hash check behind Projector.load(..., sha256)
(code/kva/integrity.py:179-198 read_verified, used by code/kva/kva.py:161-178).

A file is read once through the page cache and hashed. The reference hash is the one the caller passes
(recorded when the file was written) or, without one, the hash of the file read around the page cache
(O_DIRECT). Equal hashes: the bytes read are returned and used. Different: the file is read again around
the cache; if that copy matches the reference, the cached pages were bad (host memory), the clean copy is
returned and the file's cached pages are dropped; otherwise IntegrityError refuses the file.
"""
import errno
import hashlib
import mmap
import os
from pathlib import Path

_BLOCK = 1 << 24       # 16 MiB: a multiple of every O_DIRECT alignment


class IntegrityError(RuntimeError):
    """The file's bytes do not match its reference hash, on disk as well as in the page cache."""


def _open_uncached(path):
    """A descriptor whose reads bypass the page cache: O_DIRECT, or, on a filesystem without it, a plain
    descriptor after the file's clean cached pages have been dropped."""
    try:
        return os.open(path, os.O_RDONLY | os.O_DIRECT)
    except OSError as e:
        if e.errno != errno.EINVAL:
            raise
    fd = os.open(path, os.O_RDONLY)
    os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
    return fd


def disk_bytes(path):
    """The file's bytes as stored on disk (read around the page cache into a page-aligned buffer)."""
    fd = _open_uncached(path)
    buf = mmap.mmap(-1, _BLOCK)
    parts = []
    try:
        while True:
            n = os.readv(fd, [buf])
            if n <= 0:
                break
            parts.append(buf[:n])
    finally:
        os.close(fd)
        buf.close()
    return b"".join(parts)


def _drop_cached(path):
    fd = os.open(path, os.O_RDONLY)
    try:
        os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
    finally:
        os.close(fd)


def sha256_of(data):
    return hashlib.sha256(data).hexdigest()


def read_verified(path, ref=None):
    """(bytes, sha256 hex) of the file at path, checked against ref (a sha256 hex string, or None: the
    disk copy's hash). Raises IntegrityError when the disk copy does not match ref either."""
    path = Path(path)
    data = path.read_bytes()
    got = sha256_of(data)
    if ref is None:
        ref = sha256_of(disk_bytes(path))
    if got == ref:
        return data, got
    data = disk_bytes(path)
    got = sha256_of(data)
    if got != ref:
        raise IntegrityError(f"{path}: the file hashes to {got}, not to its reference {ref}; refusing it")
    _drop_cached(path)
    return data, got
