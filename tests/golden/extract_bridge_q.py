"""Extract the ICTC -> e3nn bridge matrix Q (lmax 4) from the reference's LAMMPS header.

lammps_user_mfftorch/src/USER-MFFTORCH/mff_mace_basis.h:15-28 holds Q_L0..Q_L4
as row-major float64 literals with x_mace = x_ictc @ Q.  The numbers are copied
into bridge_q_lmax4.json as a fixture (data only).

Usage: python tests/golden/extract_bridge_q.py /root/reference tests/golden/bridge_q_lmax4.json
"""
import json
import os
import re
import sys

ref, dest = sys.argv[1], sys.argv[2]
text = open(os.path.join(ref, "lammps_user_mfftorch", "src", "USER-MFFTORCH", "mff_mace_basis.h")).read()
body = re.search(r"Q_L4\[25\*25\] = \{([^}]*)\}", text).group(1)
values = [float(v) for v in body.split(",")]
assert len(values) == 625
json.dump({"source": "lammps_user_mfftorch/src/USER-MFFTORCH/mff_mace_basis.h:27-28 (Q_L4)",
           "lmax": 4, "row_major": values}, open(dest, "w"))
print("wrote", dest)
