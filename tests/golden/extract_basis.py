"""Extract the frozen ICTC harmonic basis (l = 0..12) as raw float64 data.

The reference ships each degree as a PyTorch zip archive whose member
``harmonic_basis_l{L}/data/0`` holds the little-endian float64 bytes of the
``[dim Sym^L, 2L+1]`` basis matrix (ictc_o3/basis/ictd_irreps.py:676-720).  The
archive is read with ``zipfile`` as bytes only (nothing is unpickled) and each
matrix is checked against the SHA-256 table of ictc_o3/basis/ictd_irreps.py:659-673
before it is written to ``harmonic_basis_v1.npz``.

Usage (in the build container, where /root/reference exists):
    python tests/golden/extract_basis.py /root/reference <out.npz>
"""
import hashlib
import os
import sys
import zipfile

import numpy as np

# ictc_o3/basis/ictd_irreps.py:659-673
SHA256 = {
    0: "6c3c396ed6b5c36dcae172271f462051b1266b851e92df3deea8ac65478fd712",
    1: "1332df685c45a61a0ac008a6a653295b8c5655361c1d34b6304b22ec40235fb8",
    2: "0881fbfd2a1866b76334d823d216ec74773a91a5f77234c45bb956838df7c315",
    3: "a7440553d51231cc044287b305d35cb5cafc59f77d7528d8189956c51a52a9e0",
    4: "f89f4b7f49ed9be8cc7fbbcec5e1a8947442c612d239bd42ce36180c6c644225",
    5: "8cce9bfb0a710f2c19d50ca3bcf6a79593697b5bd129085f10422066c2030ea8",
    6: "01cc08fe54c00daaff6899a86c923b62433f1691b7f283b95643c7be78ce9a96",
    7: "bde0ef7cf352a8cc83b4df959405616a390d270cf0b10bd93eed01da80e1a531",
    8: "85cdd2180f8078d9016110556076bf0464d12985ef079f51fee6c8f2641acf28",
    9: "190d6891295881dd5db122b80442a8feea21d0d716c6ff97faddcb0720509c6b",
    10: "fed2be677a84dc357b0e9b27e14b5bbc4c8a110520f44e536e7bc11365d70586",
    11: "4708bb0367de5a1c0d8d6bb01de80cb1a9a84ce6e128bc1913fecceabdf834ec",
    12: "761c7af5c246722d57a910b32ffe82741ac39326d6cba627be7db3b14d4ab689",
}


def extract(reference_root):
    base = os.path.join(reference_root, "ictc_o3", "basis", "_ictd_basis", "v1")
    out = {}
    for L, digest in SHA256.items():
        with zipfile.ZipFile(os.path.join(base, f"harmonic_basis_l{L}.pt")) as z:
            raw = z.read(f"harmonic_basis_l{L}/data/0")
        rows, cols = (L + 2) * (L + 1) // 2, 2 * L + 1
        if len(raw) != rows * cols * 8:
            raise RuntimeError(f"l={L}: unexpected storage size {len(raw)}")
        if hashlib.sha256(raw).hexdigest() != digest:
            raise RuntimeError(f"l={L}: SHA-256 mismatch")
        out[f"l{L}"] = np.frombuffer(raw, dtype="<f8").reshape(rows, cols).copy()
    return out


if __name__ == "__main__":
    ref, dest = sys.argv[1], sys.argv[2]
    np.savez(dest, **extract(ref))
    print("wrote", dest)
