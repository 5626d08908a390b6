"""Copy the reference test suite's weight-independent input fixtures into
tests/golden/reference_masks.npz (data only, loaded with allow_pickle=False).

Source: /root/reference/test/data/models/vlas/{pi0,pi05}/*.npy, the inputs
the reference's checkpoint-gated TestPI0FlowMatching / TestPI05FlowMatching
feed to embed_prefix / embed_suffix / make_att_2d_masks
(test/test_models/test_vla.py:253-900).  Value fixtures (embeddings,
predicted actions) depend on the pi0_base checkpoint and are not copied.

    python tests/golden/make_fixtures.py
"""
import os

import numpy as np

SRC = '/root/reference/test/data/models/vlas'
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)),
                   'reference_masks.npz')
FILES = {
    'pi0': ['prefix_pad_masks', 'prefix_att_masks', 'suffix_pad_masks',
            'suffix_att_masks', 'pad_masks', 'att_masks', 'suffix_time'],
    'pi05': ['img_masks', 'lang_masks', 'prefix_pad_masks', 'prefix_att_masks',
             'suffix_pad_masks', 'suffix_att_masks', 'suffix_time'],
}


def main():
    arrays = {}
    for d, names in FILES.items():
        for n in names:
            arrays[f'{d}_{n}'] = np.load(os.path.join(SRC, d, n + '.npy'),
                                         allow_pickle=False)
    np.savez_compressed(OUT, **arrays)
    print(f'wrote {OUT}: {sorted(arrays)}')


if __name__ == '__main__':
    main()
