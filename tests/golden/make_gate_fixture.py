"""Writes tests/golden/gate_support_sample.npz: 4096 rows of the reference's recorded router
gates (figures/allocation/support.npz: per-sample, per-level gate s (fp16), visibility and the
effective feature weight fp16(s * visible)).  Data only; run in a container that has the
reference checkout at /root/reference."""
from pathlib import Path

import numpy as np

SOURCE = Path('/root/reference/figures/allocation/support.npz')
TARGET = Path(__file__).with_name('gate_support_sample.npz')

if __name__ == '__main__':
    data = np.load(SOURCE, allow_pickle=False)
    rows = np.linspace(0, data['gate'].shape[0] - 1, 4096).astype(np.int64)
    np.savez_compressed(TARGET, gate=data['gate'][rows], visible=data['visible'][rows],
                        effective=data['effective'][rows])
    print('wrote', TARGET)
