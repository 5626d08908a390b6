"""predict_action server over the HIP inference model.

What a reference client relies on (fluxvla/engines/runners/serving/
zmq_server.py:36-284, serializers.py, proto/vla_service.proto) is the
protocol, and only that is kept:

* msgpack request ``{'endpoint': name, 'data': {...}}`` (endpoint defaults
  to predict_action) -> msgpack reply dict; endpoints ``ping`` ->
  ``{'status': 'ok', 'message': 'Server is running'}``, ``kill`` ->
  ``{'status': 'ok', 'message': 'Server shutting down'}``,
  ``predict_action(obs_data, unnorm_key)`` -> ``{'action_data': npy bytes,
  'infer_time': s}``, ``reset`` -> ``{'status': 'ok'}``, ``get_status`` ->
  ``{'status': 'ready', 'uptime_s', 'total_requests', 'avg_infer_time'}``;
  any failure -> ``{'error': message}`` (``Unknown endpoint: <name>``);
* protobuf request (0x01 tag, PredictActionRequest) -> PredictActionResponse;
  predict_action is its only call (``predict_action endpoint not
  registered`` without one).

The design is this package's own, in three parts:

* ``Call``: both wire formats parsed into one value (endpoint, keyword
  data, format); ``Call.encode(reply)`` answers in the request's format.
  A protobuf request carries a decoded observation, handed to the
  predict route as ``obs=``; a msgpack one carries ``obs_data`` bytes.
* ``PolicyServer``: a route table; ``handle(bytes) -> bytes`` answers every
  request, failures included.  The socket loop (``run``, ZMQ REP) only
  moves bytes; pyzmq is not installed in this image, so ``run`` raises
  there and every test drives ``handle``.
* ``ChunkEndpoint``: the model side -- observation -> predict_action
  inputs (``ObsToInputs``: the frames go to the GPU as uint8 and are
  resized / normalized there) -> chunk -> optional denormalization ->
  .npy bytes, with the request statistics.
"""
from __future__ import annotations
import threading
import time
from typing import Callable, NamedTuple

import numpy as np
import torch

from .serializers import (FORMAT_PROTOBUF, MsgSerializer, ObsSerializer,
                          decode_predict_request, detect_format, encode_array,
                          encode_predict_response)

PREDICT = 'predict_action'


def serialize_actions(actions: torch.Tensor) -> bytes:
    """Action tensor -> .npy bytes (the reply's action_data)."""
    return encode_array(actions.detach().cpu().numpy())


class Call(NamedTuple):
    """One parsed request: the endpoint, its keyword data, the wire format."""
    endpoint: str
    data: dict
    fmt: int

    @staticmethod
    def parse(message: bytes) -> 'Call':
        fmt = detect_format(message)
        if fmt == FORMAT_PROTOBUF:
            _, obs, unnorm_key = decode_predict_request(message)
            return Call(PREDICT, {'obs': obs, 'unnorm_key': unnorm_key}, fmt)
        request = MsgSerializer.from_bytes(message)
        return Call(request.get('endpoint', PREDICT), request.get('data', {}),
                    fmt)

    def encode(self, reply: dict) -> bytes:
        if self.fmt != FORMAT_PROTOBUF:
            return MsgSerializer.to_bytes(reply)
        if 'error' in reply:
            return encode_predict_response(b'', 0.0, FORMAT_PROTOBUF,
                                           error=reply['error'])
        return encode_predict_response(reply.get('action_data', b''),
                                       reply.get('infer_time', 0.0),
                                       FORMAT_PROTOBUF,
                                       error=reply.get('error', ''))


class _Route(NamedTuple):
    fn: Callable
    takes_data: bool


class PolicyServer:
    """Named routes answered over a ZMQ REP socket (or ``handle``)."""

    def __init__(self, host: str = '*', port: int = 5555, bind: bool = True):
        self.address = f'tcp://{host}:{port}'
        self.running = True
        self._routes: dict[str, _Route] = {
            'ping': _Route(lambda: {'status': 'ok',
                                    'message': 'Server is running'}, False),
            'kill': _Route(self._stop, False),
        }
        self._zmq = None
        if bind:
            self._open()

    def register_endpoint(self, name: str, handler: Callable,
                          requires_input: bool = True):
        """Route ``name`` to ``handler``; with ``requires_input`` the
        request's data dict is passed as keyword arguments."""
        self._routes[name] = _Route(handler, requires_input)

    def _stop(self) -> dict:
        self.running = False
        return {'status': 'ok', 'message': 'Server shutting down'}

    def _answer(self, call: Call) -> dict:
        route = self._routes.get(call.endpoint)
        if route is None:
            if call.fmt == FORMAT_PROTOBUF:
                raise LookupError(f'{PREDICT} endpoint not registered')
            raise LookupError(f'Unknown endpoint: {call.endpoint}')
        return route.fn(**call.data) if route.takes_data else route.fn()

    def handle(self, message: bytes) -> bytes:
        """One request in, one reply out (in the request's wire format);
        nothing raises past this point."""
        call = Call(PREDICT, {}, detect_format(message))
        try:
            call = Call.parse(message)
            reply = self._answer(call)
        except Exception as e:  # noqa: BLE001 -- the reply carries it
            reply = {'error': str(e)}
        return call.encode(reply)

    # -- transport ------------------------------------------------------------
    def _open(self):
        try:
            import zmq
        except ImportError as e:
            raise ImportError('PolicyServer.run needs pyzmq; without it '
                              'build the server with bind=False and call '
                              'handle(bytes)') from e
        ctx = zmq.Context()
        sock = ctx.socket(zmq.REP)
        sock.bind(self.address)
        self._zmq = (zmq, ctx, sock)

    def run(self, poll_ms: int = 500):
        """Serve until ``kill`` or ``close()``: receive, handle, send."""
        if self._zmq is None:
            self._open()
        zmq, ctx, sock = self._zmq
        print(f'Server is ready and listening on '
              f'{sock.getsockopt_string(zmq.LAST_ENDPOINT)}')
        while self.running:
            if sock.poll(poll_ms, zmq.POLLIN):
                sock.send(self.handle(sock.recv()))
        sock.setsockopt(zmq.LINGER, 0)
        sock.close()
        ctx.term()
        self._zmq = None

    def close(self):
        self.running = False


class ObsToInputs:
    """Raw observation -> predict_action keyword arguments, on the device.

    image_keys: the camera keys in view order (uint8 HWC frames, in the
    channel order the client sent them); preprocessor: an
    fluxvla_amd.preprocess.ImagePreprocessor; tokenizer / max_prompt_len:
    the prompt under ``prompt_key`` through ProcessPrompts; state_key: the
    robot state (zero-padded to state_dim)."""

    def __init__(self, image_keys, preprocessor, tokenizer=None,
                 max_prompt_len=48, prompt_key='prompt', state_key='state',
                 state_dim=32, device='cuda'):
        from ..preprocess import ProcessPrompts
        self.image_keys = list(image_keys)
        self.pre = preprocessor
        self.prompts = (ProcessPrompts(tokenizer, max_prompt_len)
                        if tokenizer is not None else None)
        self.prompt_key, self.state_key = prompt_key, state_key
        self.state_dim = state_dim
        self.device = torch.device(device)

    def __call__(self, obs: dict) -> dict:
        dev = self.device
        views = [torch.from_numpy(np.ascontiguousarray(obs[k]))[None].to(dev)
                 for k in self.image_keys]
        out = {'images': self.pre(views)}
        if self.prompts is not None:
            p = self.prompts({'prompt': obs[self.prompt_key]})
            out['lang_tokens'] = torch.from_numpy(p['lang_tokens'][None]).to(dev)
            out['lang_masks'] = torch.from_numpy(p['lang_masks'][None]).to(dev)
        else:
            out['lang_tokens'] = torch.as_tensor(obs['lang_tokens'])[None].to(dev)
            out['lang_masks'] = torch.as_tensor(obs['lang_masks'])[None].bool().to(dev)
        s = np.zeros((1, self.state_dim), np.float32)
        if self.state_key in obs:
            v = np.asarray(obs[self.state_key], np.float32).reshape(-1)
            s[0, :v.size] = v
        out['states'] = torch.from_numpy(s).to(dev)
        return out


class ChunkEndpoint:
    """The model behind the predict_action, reset and get_status routes.

    ``inputs``: observation -> predict_action keyword arguments (e.g.
    ObsToInputs, or a reference dataset pipeline, whose call may return a
    tuple led by the batch); without it the observation is the batch.
    ``denormalize``: the reference's action denormalization transform,
    called on sample 0 as ``{'action': [n, d], 'task_suite_name': ...}``."""

    def __init__(self, vla, inputs=None, denormalize=None,
                 task_suite_name: str = '', device='cuda:0'):
        self.vla, self.inputs, self.denormalize = vla, inputs, denormalize
        self.task_suite_name = task_suite_name
        self.device = torch.device(device)
        self._lock = threading.Lock()
        self._served = 0
        self._infer_s = 0.0
        self._since = time.time()

    def _batch(self, obs: dict, unnorm_key: str) -> dict:
        if self.inputs is None:
            batch = dict(obs)
        else:
            made = self.inputs(obs)
            batch = made[0] if isinstance(made, tuple) else made
        if unnorm_key:
            batch['unnorm_key'] = unnorm_key
        return {k: v.to(self.device) if isinstance(v, torch.Tensor) else v
                for k, v in batch.items()}

    def predict_action(self, obs_data: bytes = None, unnorm_key: str = '',
                       obs: dict = None) -> dict:
        if obs is None:
            obs = ObsSerializer.from_bytes(obs_data)
        batch = self._batch(obs, unnorm_key)
        t0 = time.perf_counter()
        with torch.no_grad():
            # the reply needs the values on the host: the one sync
            actions = self.vla.predict_action(**batch).cpu()
        infer_s = time.perf_counter() - t0
        if self.denormalize is not None:
            d = self.denormalize({'action': actions.numpy()[0],
                                  'task_suite_name': self.task_suite_name})
            actions = torch.from_numpy(np.asarray(d, np.float32)[None])
        with self._lock:
            self._served += 1
            self._infer_s += infer_s
        return {'action_data': serialize_actions(actions),
                'infer_time': infer_s}

    def reset(self) -> dict:
        return {'status': 'ok'}

    def get_status(self) -> dict:
        with self._lock:
            n, busy = self._served, self._infer_s
        return {'status': 'ready', 'uptime_s': time.time() - self._since,
                'total_requests': n, 'avg_infer_time': busy / n if n else 0.0}

    def attach(self, server: PolicyServer) -> PolicyServer:
        server.register_endpoint(PREDICT, self.predict_action)
        server.register_endpoint('reset', self.reset, requires_input=False)
        server.register_endpoint('get_status', self.get_status,
                                 requires_input=False)
        return server


def create_server(vla, dataset=None, denormalize_action=None,
                  task_suite_name: str = '', host: str = '*', port: int = 5555,
                  device: str = 'cuda:0', mixed_precision_dtype=None,
                  bind: bool = True) -> PolicyServer:
    """A PolicyServer serving ``vla`` with the reference's arguments
    (serve.py:121-131).  A model with ``eval`` / ``to`` (the registered
    types) is put in eval mode on ``device``.  ``mixed_precision_dtype`` is
    accepted for the reference's call and has no effect: the HIP path
    computes in bf16 with fp32 accumulation whatever autocast says."""
    for name, args in (('eval', ()), ('to', (torch.device(device),))):
        fn = getattr(vla, name, None)
        if callable(fn):
            fn(*args)
    endpoint = ChunkEndpoint(vla, dataset, denormalize_action,
                             task_suite_name, device)
    return endpoint.attach(PolicyServer(host=host, port=port, bind=bind))
