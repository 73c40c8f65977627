"""Writes tests/golden/support_storage_records.json: the per-layer support storage records
(`training.support_storage`) of every reference run under results/**/metrics.json.  Data
only; run in a container that has the reference checkout at /root/reference."""
import json
from pathlib import Path

SOURCE = Path('/root/reference/results')
TARGET = Path(__file__).with_name('support_storage_records.json')

if __name__ == '__main__':
    records = []
    for path in sorted(SOURCE.rglob('metrics.json')):
        block = json.loads(path.read_text()).get('training', {}).get('support_storage')
        if block:
            records.append(dict(run=str(path.relative_to(SOURCE)), **block))
    TARGET.write_text(json.dumps(records, indent=1) + '\n')
    print('wrote', TARGET, len(records), 'runs')
