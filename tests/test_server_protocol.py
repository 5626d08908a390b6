"""The server's protocol replies on the CPU (no model): the reply strings
and keys a reference client reads (zmq_server.py:36-284), in both wire
formats, and the endpoint object's statistics."""
import io

import numpy as np
import torch

from fluxvla_amd.serving import serializers as S
from fluxvla_amd.serving.server import ChunkEndpoint, PolicyServer


def _msg(srv, req):
    return S.MsgSerializer.from_bytes(srv.handle(S.MsgSerializer.to_bytes(req)))


def test_builtin_routes_and_errors_without_a_model():
    srv = PolicyServer(bind=False)
    assert _msg(srv, {'endpoint': 'ping'}) == {'status': 'ok',
                                               'message': 'Server is running'}
    # the default endpoint is predict_action, not registered here
    assert _msg(srv, {'data': {}}) == {
        'error': 'Unknown endpoint: predict_action'}
    raw = S.encode_predict_request({'state': np.zeros(2, np.float32)}, '',
                                   fmt='protobuf')
    assert S.decode_predict_response(srv.handle(raw), S.FORMAT_PROTOBUF) == {
        'error': 'predict_action endpoint not registered'}
    # undecodable protobuf bytes are answered in protobuf
    resp = S.decode_predict_response(srv.handle(b'\x01\xff\xff'),
                                     S.FORMAT_PROTOBUF)
    assert 'error' in resp
    assert _msg(srv, {'endpoint': 'kill'}) == {
        'status': 'ok', 'message': 'Server shutting down'}
    assert not srv.running


class _Echo:
    def predict_action(self, state, **kw):
        return torch.as_tensor(state, dtype=torch.float32)[None, None].repeat(
            1, 3, 1)


def test_endpoint_statistics_and_denormalization():
    seen = []

    def denorm(d):
        seen.append(d['task_suite_name'])
        return d['action'] * 10
    ep = ChunkEndpoint(_Echo(), denormalize=denorm, task_suite_name='libero',
                       device='cpu')
    srv = ep.attach(PolicyServer(bind=False))
    st = np.array([1.0, 2.0], np.float32)
    raw = S.encode_predict_request({'state': st}, '')
    acts = np.load(io.BytesIO(S.decode_predict_response(srv.handle(raw))[
        'action_data']))
    assert acts.shape == (1, 3, 2) and np.all(acts == 10 * st)
    assert seen == ['libero']
    status = _msg(srv, {'endpoint': 'get_status'})
    assert status['status'] == 'ready' and status['total_requests'] == 1
    assert status['avg_infer_time'] >= 0.0 and status['uptime_s'] >= 0.0
    assert _msg(srv, {'endpoint': 'reset'}) == {'status': 'ok'}


def test_inputs_pipeline_may_return_a_tuple():
    """A reference dataset pipeline returns (batch, ...): the batch is its
    first element."""
    ep = ChunkEndpoint(_Echo(), inputs=lambda obs: ({'state': obs['s']}, None),
                       device='cpu')
    out = ep.predict_action(obs={'s': np.ones(4, np.float32)})
    acts = np.load(io.BytesIO(out['action_data']))
    assert acts.shape == (1, 3, 4)
