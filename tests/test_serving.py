"""Serving boundary on the CPU: wire formats against known-answer bytes of
the reference's schema (fluxvla/engines/runners/serving/serializers.py,
proto/vla_service.proto) and the endpoint dispatch of PolicyServer
(zmq_server.py:36-284) with a stand-in model."""
import io
import struct

import msgpack
import numpy as np
import pytest
import torch

from fluxvla_amd.serving import serializers as S
from fluxvla_amd.serving.server import PolicyServer, create_server


def test_protobuf_response_known_bytes():
    """PredictActionResponse{action_data=b'ab', infer_time=0.5}: field 1
    bytes (tag 0x0a), field 2 double (tag 0x11), behind the 0x01 tag."""
    raw = S.encode_predict_response(b'ab', 0.5, S.FORMAT_PROTOBUF)
    assert raw == b'\x01\x0a\x02ab\x11' + struct.pack('<d', 0.5)
    err = S.encode_predict_response(b'', 0.0, S.FORMAT_PROTOBUF, error='x')
    assert err == b'\x01\x1a\x01x'  # field 3 string
    assert S.decode_predict_response(raw, S.FORMAT_PROTOBUF) == {
        'action_data': b'ab', 'infer_time': 0.5}
    assert S.decode_predict_response(err, S.FORMAT_PROTOBUF) == {'error': 'x'}


def test_protobuf_request_known_bytes():
    """PredictActionRequest{obs{strings{'p': 'q'}}, unnorm_key='u'}: the
    map entry is a nested message {key=1, value=2} under Observation field
    3, the observation under request field 1, the key under field 2."""
    raw = S.encode_predict_request({'p': 'q'}, 'u', fmt='protobuf')
    entry = b'\x0a\x01p\x12\x01q'
    obs = b'\x1a' + bytes([len(entry)]) + entry
    assert raw == b'\x01\x0a' + bytes([len(obs)]) + obs + b'\x12\x01u'
    fmt, o, key = S.decode_predict_request(raw)
    assert (fmt, o, key) == (S.FORMAT_PROTOBUF, {'p': 'q'}, 'u')
    arr = np.arange(6, dtype=np.float32).reshape(2, 3)
    raw = S.encode_predict_request({'state': arr}, '', fmt='protobuf')
    _, o, _ = S.decode_predict_request(raw)
    assert np.array_equal(o['state'], arr)


def test_msgpack_request_layout():
    """{'endpoint': 'predict_action', 'data': {'obs_data': msgpack map,
    'unnorm_key': ...}} with __jpeg__ / __ndarray__ / plain string values."""
    img = np.zeros((16, 16, 3), np.uint8)
    st = np.ones(14, np.float32)
    raw = S.encode_predict_request({'cam_high': img, 'state': st,
                                    'prompt': 'go'}, 'aloha')
    outer = msgpack.unpackb(raw, raw=False)
    assert outer['endpoint'] == 'predict_action'
    assert outer['data']['unnorm_key'] == 'aloha'
    inner = msgpack.unpackb(outer['data']['obs_data'], raw=False)
    assert inner['cam_high']['__jpeg__'] is True
    assert inner['cam_high']['data'][:2] == b'\xff\xd8'  # JPEG SOI
    assert inner['state']['__ndarray__'] is True
    assert np.array_equal(np.load(io.BytesIO(inner['state']['data'])), st)
    assert inner['prompt'] == 'go'
    fmt, obs, key = S.decode_predict_request(raw)
    assert fmt == S.FORMAT_MSGPACK and key == 'aloha'
    assert obs['cam_high'].shape == (16, 16, 3) and obs['prompt'] == 'go'


def test_jpeg_keeps_channel_order():
    """A frame round trips in the caller's channel order (what OpenCV's
    BGR encode / decode pair does)."""
    img = np.zeros((64, 64, 3), np.uint8)
    img[:, :, 0] = 200
    img[:, :, 2] = 30
    back = S.decode_image(S.encode_image(img))
    assert np.abs(back.astype(int) - img).max() <= 3


class _Fake:
    """Stand-in model: returns a chunk that encodes its inputs."""

    def __init__(self):
        self.calls = []

    def predict_action(self, **batch):
        self.calls.append(batch)
        s = torch.as_tensor(batch['state'], dtype=torch.float32)
        return s.sum() * torch.ones(1, 50, 32)


def test_server_endpoints_and_errors():
    vla = _Fake()
    srv = create_server(vla, device='cpu', bind=False)
    ping = MsgSerializer_roundtrip(srv, {'endpoint': 'ping'})
    assert ping['status'] == 'ok'
    assert 'Unknown endpoint' in MsgSerializer_roundtrip(
        srv, {'endpoint': 'nope'})['error']
    raw = S.encode_predict_request({'state': np.full(4, 2.0, np.float32)}, '')
    resp = S.decode_predict_response(srv.handle(raw))
    acts = np.load(io.BytesIO(resp['action_data']))
    assert acts.shape == (1, 50, 32) and np.all(acts == 8.0)
    assert resp['infer_time'] >= 0.0
    # protobuf predict path
    raw = S.encode_predict_request({'state': np.full(4, 1.0, np.float32)}, 'k',
                                   fmt='protobuf')
    resp = S.decode_predict_response(srv.handle(raw), S.FORMAT_PROTOBUF)
    assert np.all(np.load(io.BytesIO(resp['action_data'])) == 4.0)
    assert vla.calls[-1]['unnorm_key'] == 'k'
    st = MsgSerializer_roundtrip(srv, {'endpoint': 'get_status'})
    assert st['total_requests'] == 2
    # a failing model replies with the error instead of raising
    bad = S.encode_predict_request({'other': np.zeros(2, np.float32)}, '')
    assert 'state' in S.decode_predict_response(srv.handle(bad))['error']
    assert MsgSerializer_roundtrip(srv, {'endpoint': 'kill'})['status'] == 'ok'
    assert not srv.running


def MsgSerializer_roundtrip(srv, req):
    return S.MsgSerializer.from_bytes(srv.handle(S.MsgSerializer.to_bytes(req)))


def test_run_needs_pyzmq():
    try:
        import zmq  # noqa: F401
        pytest.skip('pyzmq is installed')
    except ImportError:
        with pytest.raises(ImportError):
            PolicyServer(bind=True)


def test_msgpack_observation_bytes_and_order():
    """The reference's map order (frames, then arrays, then strings, each
    in the observation's order) and bytes; untagged values pass through."""
    img = np.zeros((8, 8, 3), np.uint8)
    st = np.arange(3, dtype=np.float32)
    obs = {'prompt': 'go', 'state': st, 'cam_high': img}
    raw = S.ObsSerializer.to_bytes(obs)
    npy = io.BytesIO()
    np.save(npy, st, allow_pickle=False)
    want_tail = msgpack.packb({'state': {'__ndarray__': True,
                                         'data': npy.getvalue()},
                               'prompt': 'go'})
    keys = list(msgpack.unpackb(raw, raw=False))
    assert keys == ['cam_high', 'state', 'prompt']
    # the map after its first entry is byte for byte the arrays and strings
    assert raw.endswith(want_tail[1:])
    extra = msgpack.packb({'meta': {'a': 1}, 'name': b'xy'})
    assert S.ObsSerializer.from_bytes(extra) == {'meta': {'a': 1},
                                                 'name': 'xy'}
    back = S.ObsSerializer.from_bytes(raw)
    assert list(back) == keys and back['prompt'] == 'go'
    assert np.array_equal(back['state'], st) and back['cam_high'].shape == (8, 8, 3)
    assert S.MsgSerializer.from_bytes(S.MsgSerializer.to_bytes(
        {'x': [st, 1]}))['x'][0].tolist() == [0.0, 1.0, 2.0]
