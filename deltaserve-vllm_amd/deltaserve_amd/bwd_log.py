"""The parent's per-cycle ``bwd_log.csv`` row (coordinator.py:1079-1109 of the
reference): timestamp, epoch, batch_idx, batch_tokens, batch_loss,
total_processed_tokens; the header is written to a new or empty file."""

from __future__ import annotations

import csv
import datetime
import os

HEADER = ["timestamp", "epoch", "batch_idx", "batch_tokens", "batch_loss",
          "total_processed_tokens"]


class BwdLog:
    def __init__(self, path: str) -> None:
        self.path = path
        self.batch_idx = 0
        self.total_tokens = 0

    def write_row(self, epoch: int, n: int, loss) -> None:
        self.batch_idx += 1
        self.total_tokens += int(n)
        parent = os.path.dirname(self.path)
        if parent:
            os.makedirs(parent, exist_ok=True)
        new_file = not os.path.exists(self.path) or os.path.getsize(self.path) == 0
        with open(self.path, "a", newline="") as f:
            w = csv.writer(f)
            if new_file:
                w.writerow(HEADER)
            w.writerow([datetime.datetime.now().isoformat(timespec="milliseconds"), int(epoch),
                        self.batch_idx, int(n), "" if loss is None else loss,
                        self.total_tokens])
