"""Token alphabets of ESM-2 / MINT (the index layout of
``mint_plus/models/alphabet.py:4-73``): special tokens first, the protein
tokens, ``<null_i>`` filler up to a multiple of 8, then the appended tokens.
Only the index bookkeeping the model needs (no tokenizer)."""
from typing import Sequence

PROTEIN_TOKS = ("L", "A", "G", "V", "S", "E", "R", "T", "I", "D", "P", "K", "Q", "N", "F", "Y",
                "M", "H", "W", "C", "X", "B", "U", "Z", "O", ".", "-")
STANDARD_AA = PROTEIN_TOKS[:20]


class Alphabet:
    def __init__(self, standard_toks: Sequence[str],
                 prepend_toks: Sequence[str] = ("<null_0>", "<pad>", "<eos>", "<unk>"),
                 append_toks: Sequence[str] = ("<cls>", "<mask>", "<sep>"),
                 prepend_bos: bool = True, append_eos: bool = False):
        self.standard_toks = list(standard_toks)
        self.prepend_toks = list(prepend_toks)
        self.append_toks = list(append_toks)
        self.prepend_bos = prepend_bos
        self.append_eos = append_eos
        toks = self.prepend_toks + self.standard_toks
        toks += [f"<null_{i + 1}>" for i in range(-len(toks) % 8)]
        self.all_toks = toks + self.append_toks
        self.tok_to_idx = {t: i for i, t in enumerate(self.all_toks)}
        self.unk_idx = self.tok_to_idx["<unk>"]
        self.padding_idx = self.tok_to_idx["<pad>"]
        self.cls_idx = self.tok_to_idx["<cls>"]
        self.mask_idx = self.tok_to_idx["<mask>"]
        self.eos_idx = self.tok_to_idx["<eos>"]

    def __len__(self):
        return len(self.all_toks)

    def get_idx(self, tok):
        return self.tok_to_idx.get(tok, self.unk_idx)

    def get_tok(self, ind):
        return self.all_toks[ind]

    @classmethod
    def from_architecture(cls, name: str) -> "Alphabet":
        if name in ("ESM-1", "protein_bert_base"):
            return cls(PROTEIN_TOKS, ("<null_0>", "<pad>", "<eos>", "<unk>"),
                       ("<cls>", "<mask>", "<sep>"), True, False)
        if name in ("ESM-1b", "roberta_large"):
            return cls(PROTEIN_TOKS, ("<cls>", "<pad>", "<eos>", "<unk>"), ("<mask>",), True, True)
        raise ValueError(f"Unknown architecture: {name}")
