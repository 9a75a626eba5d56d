"""HalfKAv2_hm^ feature block (reference src/model/modules/features/halfka_v2_hm.py:40-193).

Rows: 12 piece planes x 64 squares x 32 king buckets = 24 576, plus 768
"virtual" factor rows shared by all buckets.  The table the FT reads is
`weight + virtual_weight` tiled over the 32 buckets (row r gets virtual row
r mod 768).  Export folds the two king planes into one (11 planes, 22 528 rows).

Square numbering is a1 = 0 .. h8 = 63.  The horizontal-mirror orientation puts
the own king on files e-h; the king bucket of an oriented king square on rank r,
file f (f >= 4) is (7 - r) * 4 + (7 - f).
"""

import torch
from torch import nn

from .input_feature import InputFeature

# python-chess piece-type codes (PAWN=1 .. KING=6) and the material values the
# reference seeds its PSQT columns with (halfka_v2_hm.py:174-180).
PAWN, KNIGHT, BISHOP, ROOK, QUEEN, KING = 1, 2, 3, 4, 5, 6
_PSQT_PIECE_VALUES = {PAWN: 126, KNIGHT: 781, BISHOP: 825, ROOK: 1276, QUEEN: 2538}


def king_bucket(oriented_ksq: int) -> int:
    rank, file = divmod(oriented_ksq, 8)
    return -1 if file < 4 else (7 - rank) * 4 + (7 - file)


KingBuckets = [king_bucket(sq) for sq in range(64)]
InverseKingBuckets = [0] * 32
for _sq, _b in enumerate(KingBuckets):
    if _b >= 0:
        InverseKingBuckets[_b] = _sq


def _orient(white_pov: bool, sq: int, ksq: int) -> int:
    flip_file = 7 if (ksq % 8) < 4 else 0
    flip_rank = 0 if white_pov else 56
    return sq ^ flip_file ^ flip_rank


def halfka_index(white_pov: bool, king_sq: int, sq: int, piece_type: int, piece_white: bool) -> int:
    """Training index of a piece (12 planes, own king not merged)."""
    plane = (piece_type - 1) * 2 + (0 if piece_white == white_pov else 1)
    bucket = KingBuckets[_orient(white_pov, king_sq, king_sq)]
    return _orient(white_pov, sq, king_sq) + 64 * plane + 768 * bucket


class HalfKav2Hm(InputFeature):
    HASH = 0x7F234CB8
    FEATURE_NAME = "HalfKAv2_hm^"
    INPUT_FEATURE_NAME = "HalfKAv2_hm"
    MAX_ACTIVE_FEATURES = 32

    NUM_SQ = 64
    NUM_PT = 12
    NUM_PLANES = NUM_SQ * NUM_PT  # 768
    NUM_BUCKETS = NUM_SQ // 2  # 32
    NUM_INPUTS = NUM_PLANES * NUM_BUCKETS  # 24 576
    NUM_INPUTS_VIRTUAL = NUM_PLANES  # 768
    NUM_REAL_FEATURES = 704 * 32  # 22 528 exported rows (11 planes)

    def __init__(self, num_outputs: int):
        super().__init__()
        self.num_outputs = num_outputs
        self.weight = nn.Parameter(torch.empty(self.NUM_INPUTS, num_outputs, dtype=torch.float32))
        self.virtual_weight = nn.Parameter(
            torch.zeros(self.NUM_INPUTS_VIRTUAL, num_outputs, dtype=torch.float32))
        self.reset_parameters()

    def merged_weight(self) -> torch.Tensor:
        return self.weight + self.virtual_weight.repeat(self.NUM_BUCKETS, 1)

    def table_blocks(self):
        return self.weight, self.virtual_weight

    @torch.no_grad()
    def coalesce(self) -> None:
        self.weight.add_(self.virtual_weight.repeat(self.NUM_BUCKETS, 1))
        self.virtual_weight.zero_()

    @torch.no_grad()
    def init_weights(self, num_psqt_buckets: int, nnue2score: float) -> None:
        """Zero the virtual rows and seed every PSQT column with material / nnue2score."""
        self.virtual_weight.zero_()
        values = torch.tensor(self.halfka_psqts(), dtype=self.weight.dtype, device=self.weight.device)
        values = values * (1.0 / nnue2score)
        first = self.num_outputs - num_psqt_buckets
        for col in range(first, self.num_outputs):
            self.weight[:, col] = values

    @torch.no_grad()
    def get_export_weights(self) -> torch.Tensor:
        """Coalesced table with the two king planes of each bucket folded into one."""
        full = self.weight.detach() + self.virtual_weight.detach().repeat(self.NUM_BUCKETS, 1)
        per_bucket = full.view(self.NUM_BUCKETS, self.NUM_PLANES, -1)
        out = full.new_zeros(self.NUM_BUCKETS, 704, full.shape[1])
        out[:, :640] = per_bucket[:, :640]  # planes 0..9
        out[:, 640:704] = per_bucket[:, 704:768]  # opponent king plane
        for b in range(self.NUM_BUCKETS):
            ksq = InverseKingBuckets[b]
            out[b, 640 + ksq] = per_bucket[b, 640 + ksq]  # own king on its bucket square
        return out.reshape(self.NUM_REAL_FEATURES, -1)

    @torch.no_grad()
    def load_export_weights(self, export_weight: torch.Tensor) -> None:
        src = export_weight.view(self.NUM_BUCKETS, 704, -1)
        full = export_weight.new_zeros(self.NUM_BUCKETS, self.NUM_PLANES, export_weight.shape[1])
        full[:, :640] = src[:, :640]
        full[:, 704:768] = src[:, 640:704]
        for b in range(self.NUM_BUCKETS):
            ksq = InverseKingBuckets[b]
            full[b, 640 + ksq] = src[b, 640 + ksq]
            full[b, 704 + ksq] = 0
        self.weight.copy_(full.view(self.NUM_INPUTS, -1))
        self.virtual_weight.zero_()

    @staticmethod
    def halfka_psqts() -> list:
        """Material value of every training row seen from White (kings 0)."""
        values = [0] * (768 * 32)
        for ksq in range(64):
            for sq in range(64):
                for pt, val in _PSQT_PIECE_VALUES.items():
                    values[halfka_index(True, ksq, sq, pt, True)] = val
                    values[halfka_index(True, ksq, sq, pt, False)] = -val
        return values
