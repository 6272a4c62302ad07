"""Pack a solution folder into solution.json (the counterpart of the
reference's scripts/pack_solution.py).

Usage:
    python gated-delta-network_amd/solutions/pack_solution.py gdn_decode_qk4_v8_d128_k_last
    python gated-delta-network_amd/solutions/pack_solution.py all
"""

import os
import sys

sys.path.insert(0, os.path.abspath(os.path.join(os.path.dirname(__file__), os.pardir)))

from gdn_amd.packing import main  # noqa: E402

if __name__ == "__main__":
    sys.exit(main())
