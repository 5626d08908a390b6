"""The predict_action endpoint end to end on the GPU: a JPEG/msgpack (and
protobuf) request through PolicyServer.handle, device preprocessing and the
chunk graph, against the CPU oracle on the host transforms' images."""
import io

import numpy as np
import pytest
import torch

from fluxvla_amd.serving import serializers as S
from oracle import preprocess_oracle as PO
from tests.conftest import announce

pytestmark = pytest.mark.gpu

MEANS = [[123.515625, 116.04492188, 103.59375]] * 3
STDS = [[58.27148438, 57.02636719, 57.27539062]] * 3
CAMS = ['cam_high', 'cam_left_wrist', 'cam_right_wrist']


def test_predict_action_request_end_to_end(cuda):
    announce('serving predict_action msgpack + protobuf')
    from fluxvla_amd.config import tiny
    from fluxvla_amd.pi0_inference import PI0Inference
    from fluxvla_amd.preprocess import ImagePreprocessor
    from fluxvla_amd.serving.server import ObsToInputs, create_server
    from fluxvla_amd.weights import make_inputs, make_state_dict
    from oracle import pi0_oracle as O
    cfg = tiny(vit_layers=1, llm_layers=1, exp_layers=1)
    sd = make_state_dict(cfg, seed=8)
    m = PI0Inference(cfg, sd, device='cuda')
    inp = make_inputs(cfg, batch=1, seed=9)
    g = torch.Generator().manual_seed(10)
    obs = {c: torch.randint(0, 256, (480, 640, 3), generator=g,
                            dtype=torch.uint8).numpy() for c in CAMS}
    obs['state'] = inp['states'][0].numpy()
    obs['lang_tokens'] = inp['lang_tokens'][0].numpy()
    obs['lang_masks'] = inp['lang_masks'][0].numpy()
    pre = ImagePreprocessor.from_transforms([
        dict(type='ResizeImages', height=224, width=224),
        dict(type='NormalizeImages', means=MEANS, stds=STDS)])
    ds = ObsToInputs(CAMS, pre, device=cuda)

    def with_noise(o):
        b = ds(o)
        b['noise'] = inp['noise'].to(cuda)
        return b

    srv = create_server(m, dataset=with_noise, device=str(cuda), bind=False)
    resp = S.decode_predict_response(srv.handle(S.encode_predict_request(obs, '')))
    assert 'error' not in resp, resp.get('error')
    acts = np.load(io.BytesIO(resp['action_data']))
    presp = S.decode_predict_response(
        srv.handle(S.encode_predict_request(obs, '', fmt='protobuf')),
        S.FORMAT_PROTOBUF)
    assert np.array_equal(np.load(io.BytesIO(presp['action_data'])), acts)
    # oracle: the frames as the server decodes them, host transforms
    dec = {c: S.decode_image(S.encode_image(obs[c])) for c in CAMS}
    r8 = np.stack([PO.resize_linear_u8(dec[c], 224, 224).transpose(2, 0, 1)
                   for c in CAMS])
    imgs = torch.from_numpy(PO.normalize_images(r8, MEANS, STDS)).reshape(
        1, 9, 224, 224)
    ref = O.predict_action(sd, cfg, imgs, inp['lang_tokens'], inp['states'],
                           noise=inp['noise'])
    err = np.abs(acts - ref.numpy()).max()
    print(f'served chunk max abs err vs oracle {err:.3e}, '
          f'infer {resp["infer_time"] * 1e3:.2f} ms')
    assert err <= 2e-2
