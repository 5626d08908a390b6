"""predict_action server over the HIP inference model.

Mirrors the reference's two layers (fluxvla/engines/runners/serving/
zmq_server.py:36-284): PolicyServer routes named endpoints (ping, kill,
predict_action, reset, get_status) for msgpack requests and answers 0x01
protobuf requests on the predict path; create_server wires a VLA into it.

The transport is separate from the dispatch: ``handle(message) -> reply``
is the whole request/reply step, and ``run()`` drives it from a ZMQ REP
socket as the reference does.  pyzmq is not installed in this image, so
``run()`` raises there, and every test goes through ``handle``.

On this path the observation's frames go to the GPU as uint8 and are resized
and normalized there (fluxvla_amd.preprocess), instead of through the
host-side transform chain the reference runs before predict_action.
"""
from __future__ import annotations
import threading
import time
from dataclasses import dataclass
from typing import Callable

import numpy as np
import torch

from .serializers import (FORMAT_PROTOBUF, MsgSerializer, ObsSerializer,
                          decode_predict_request, detect_format, encode_array,
                          encode_predict_response)


def serialize_actions(actions: torch.Tensor) -> bytes:
    """Action tensor -> .npy bytes (zmq_server.py:29-32)."""
    return encode_array(actions.detach().cpu().numpy())


@dataclass
class EndpointHandler:
    handler: Callable
    requires_input: bool = True


class PolicyServer:
    """Named-endpoint request/reply server (zmq_server.py:36-176)."""

    def __init__(self, host: str = '*', port: int = 5555, bind: bool = True):
        self.running = True
        self.host, self.port = host, port
        self._endpoints: dict[str, EndpointHandler] = {}
        self.register_endpoint('ping', self._handle_ping, requires_input=False)
        self.register_endpoint('kill', self._kill_server, requires_input=False)
        self.socket = self.context = None
        if bind:
            self._bind()

    def _bind(self):
        try:
            import zmq
        except ImportError as e:
            raise ImportError('PolicyServer.run needs pyzmq; dispatch a '
                              'request with PolicyServer.handle(bytes) '
                              'without it (bind=False)') from e
        self.context = zmq.Context()
        self.socket = self.context.socket(zmq.REP)
        self.socket.bind(f'tcp://{self.host}:{self.port}')

    def register_endpoint(self, name: str, handler: Callable,
                          requires_input: bool = True):
        self._endpoints[name] = EndpointHandler(handler, requires_input)

    def _handle_ping(self) -> dict:
        return {'status': 'ok', 'message': 'Server is running'}

    def _kill_server(self):
        self.running = False
        return {'status': 'ok', 'message': 'Server shutting down'}

    def handle(self, message: bytes) -> bytes:
        """One request -> one reply.  Errors are replied, never raised
        (zmq_server.py:115-136, 142-176)."""
        if detect_format(message) == FORMAT_PROTOBUF:
            return self._handle_protobuf_predict(message)
        try:
            request = MsgSerializer.from_bytes(message)
            endpoint = request.get('endpoint', 'predict_action')
            if endpoint not in self._endpoints:
                raise ValueError(f'Unknown endpoint: {endpoint}')
            h = self._endpoints[endpoint]
            result = (h.handler(**request.get('data', {}))
                      if h.requires_input else h.handler())
            return MsgSerializer.to_bytes(result)
        except Exception as e:  # noqa: BLE001 -- the reply carries it
            return MsgSerializer.to_bytes({'error': str(e)})

    def _handle_protobuf_predict(self, message: bytes) -> bytes:
        try:
            _, obs, unnorm_key = decode_predict_request(message)
            h = self._endpoints.get('predict_action')
            if h is None:
                return encode_predict_response(
                    b'', 0.0, FORMAT_PROTOBUF,
                    error='predict_action endpoint not registered')
            result = h.handler(obs_data=None, unnorm_key=unnorm_key,
                               _obs_dict=obs, _wire_format=FORMAT_PROTOBUF)
            return encode_predict_response(result.get('action_data', b''),
                                           result.get('infer_time', 0.0),
                                           FORMAT_PROTOBUF,
                                           error=result.get('error', ''))
        except Exception as e:  # noqa: BLE001
            return encode_predict_response(b'', 0.0, FORMAT_PROTOBUF, error=str(e))

    def run(self):
        """Blocking ZMQ REP loop until ``kill`` or ``close()``."""
        import zmq
        if self.socket is None:
            self._bind()
        print(f'Server is ready and listening on '
              f'{self.socket.getsockopt_string(zmq.LAST_ENDPOINT)}')
        poller = zmq.Poller()
        poller.register(self.socket, zmq.POLLIN)
        while self.running:
            if self.socket in dict(poller.poll(timeout=500)):
                self.socket.send(self.handle(self.socket.recv()))
        self.socket.setsockopt(zmq.LINGER, 0)
        self.socket.close()
        self.context.term()

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


def create_server(vla, dataset=None, denormalize_action=None,
                  task_suite_name: str = '', host: str = '*', port: int = 5555,
                  device: str = 'cuda:0', bind: bool = True) -> PolicyServer:
    """A PolicyServer around ``vla`` (zmq_server.py:179-284).  ``dataset``:
    callable observation -> predict_action kwargs (e.g. ObsToInputs);
    ``denormalize_action``: the reference's action denormalization
    transform.  The reference's autocast is not needed: the HIP path
    computes in bf16 with fp32 accumulation by construction."""
    dev = torch.device(device)
    lock = threading.Lock()
    stats = {'n': 0, 'infer': 0.0, 'start': time.time()}

    def predict_action(obs_data: bytes = None, unnorm_key: str = '',
                       _obs_dict: dict = None, _wire_format: int = 0) -> dict:
        obs = _obs_dict if _obs_dict is not None else ObsSerializer.from_bytes(obs_data)
        if dataset is not None:
            result = dataset(obs)
            batch = result[0] if isinstance(result, tuple) else result
        else:
            batch = obs
        if unnorm_key:
            batch['unnorm_key'] = unnorm_key
        t0 = time.perf_counter()
        with torch.no_grad():
            for k, v in batch.items():
                if isinstance(v, torch.Tensor):
                    batch[k] = v.to(dev)
            actions = vla.predict_action(**batch)
            actions = actions.cpu()  # the reply needs the values: one sync
        infer_time = time.perf_counter() - t0
        if denormalize_action is not None:
            d = denormalize_action(dict(action=actions.numpy()[0],
                                        task_suite_name=task_suite_name))
            actions = torch.from_numpy(d[None].astype(np.float32))
        with lock:
            stats['n'] += 1
            stats['infer'] += infer_time
        return {'action_data': serialize_actions(actions),
                'infer_time': infer_time}

    def reset() -> dict:
        return {'status': 'ok'}

    def get_status() -> dict:
        with lock:
            n = stats['n']
            avg = stats['infer'] / n if n else 0.0
        return {'status': 'ready', 'uptime_s': time.time() - stats['start'],
                'total_requests': n, 'avg_infer_time': avg}

    server = PolicyServer(host=host, port=port, bind=bind)
    server.register_endpoint('predict_action', predict_action)
    server.register_endpoint('reset', reset, requires_input=False)
    server.register_endpoint('get_status', get_status, requires_input=False)
    return server
