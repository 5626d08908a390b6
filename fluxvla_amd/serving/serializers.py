"""Wire formats of the predict_action endpoint.

Byte-compatible with the reference's serializers
(fluxvla/engines/runners/serving/serializers.py:1-250) and its protobuf
schema (serving/proto/vla_service.proto), so a reference client talks to
this server unchanged.  What the bytes are:

* msgpack (default): ``{"endpoint": name, "data": {...}}``; an observation is
  a msgpack map whose values are ``{"__jpeg__": True, "data": jpeg}`` for
  compressed camera frames, ``{"__ndarray__": True, "data": npy}`` for
  arrays, or plain strings (frames first, then arrays, then strings);
  responses carry the action tensor as .npy bytes.
* protobuf: first byte 0x01, then a PredictActionRequest /
  PredictActionResponse message.  The message classes are built at import
  from a descriptor equal to vla_service.proto (no generated code needed).

How this module is arranged: every observation value is classified once
into one of the three payload kinds of the schema (``images`` / ``arrays``
/ ``strings``, also the names of the Observation message's maps), and both
wire formats are views of that split; replies are plain dicts that either
format encodes.  The reference's class and function names are kept as the
client-facing API (a client imports ``encode_predict_request``,
``ObsSerializer``, ...).

JPEG: the reference encodes and decodes with OpenCV, which treats the
three channels as B, G, R.  OpenCV is not installed here; Pillow does the
coding with the channel order reversed on both sides, so a frame round
trips in the caller's channel order and the JPEG stream means what an
OpenCV client's stream means.
"""
from __future__ import annotations
import io
from concurrent.futures import ThreadPoolExecutor
from typing import Any

import msgpack
import numpy as np

# protocol constants (the reference's values)
FORMAT_MSGPACK: int = 0x00
FORMAT_PROTOBUF: int = 0x01
JPEG_QUALITY = 95
JPEG_KEYS = frozenset({
    'cam_high', 'cam_left_wrist', 'cam_right_wrist', 'agentview_image',
    'robot0_eye_in_hand_image',
})

# payload kinds, in wire order; each is also an Observation map's name
IMAGES, ARRAYS, STRINGS = 'images', 'arrays', 'strings'
KINDS = (IMAGES, ARRAYS, STRINGS)
# the msgpack envelope key of a kind (strings travel bare)
_ENVELOPE = {IMAGES: '__jpeg__', ARRAYS: '__ndarray__'}


def detect_format(raw: bytes) -> int:
    """0x01 first byte: protobuf; anything else: msgpack."""
    return FORMAT_PROTOBUF if raw[:1] == b'\x01' else FORMAT_MSGPACK


# ---------------------------------------------------------------------------
# payload codecs
# ---------------------------------------------------------------------------
def encode_image(img: np.ndarray) -> bytes:
    """uint8 [h, w, 3] in OpenCV's B, G, R order -> JPEG (quality 95)."""
    from PIL import Image
    buf = io.BytesIO()
    Image.fromarray(np.ascontiguousarray(img[:, :, ::-1])).save(
        buf, format='JPEG', quality=JPEG_QUALITY)
    return buf.getvalue()


def decode_image(data: bytes) -> np.ndarray:
    """JPEG -> uint8 [h, w, 3] in B, G, R order (cv2.imdecode IMREAD_COLOR)."""
    from PIL import Image
    img = Image.open(io.BytesIO(data)).convert('RGB')
    return np.ascontiguousarray(np.asarray(img)[:, :, ::-1])


_POOL = None


def decode_images(blobs: dict) -> dict:
    """Decode several JPEG frames at once: the codec releases the GIL, so
    the camera views decode on parallel host threads (the reference decodes
    them one after another)."""
    global _POOL
    if len(blobs) < 2:
        return {k: decode_image(v) for k, v in blobs.items()}
    if _POOL is None:
        _POOL = ThreadPoolExecutor(max_workers=4, thread_name_prefix='jpeg')
    keys = list(blobs)
    return dict(zip(keys, _POOL.map(decode_image, [blobs[k] for k in keys])))


def encode_array(arr: np.ndarray) -> bytes:
    """ndarray -> .npy bytes (no pickles)."""
    buf = io.BytesIO()
    np.save(buf, arr, allow_pickle=False)
    return buf.getvalue()


def decode_array(data: bytes) -> np.ndarray:
    return np.load(io.BytesIO(data), allow_pickle=False)


# ---------------------------------------------------------------------------
# observations: one split, two wire views
# ---------------------------------------------------------------------------
def _kind_of(key: str, value, compress: bool):
    """The payload kind a value travels as, or None (not sent)."""
    if isinstance(value, np.ndarray):
        frame = value.ndim == 3 and value.dtype == np.uint8
        return IMAGES if compress and frame and key in JPEG_KEYS else ARRAYS
    return STRINGS if isinstance(value, str) else None


_TO_PAYLOAD = {IMAGES: encode_image, ARRAYS: encode_array, STRINGS: str}


def split_observation(obs: dict, compress: bool = True) -> dict:
    """{kind: {key: payload}} of an observation (JPEG bytes, .npy bytes,
    strings), each kind in the observation's key order."""
    parts = {k: {} for k in KINDS}
    for key, value in obs.items():
        kind = _kind_of(key, value, compress)
        if kind is not None:
            parts[kind][key] = _TO_PAYLOAD[kind](value)
    return parts


def join_observation(parts: dict) -> dict:
    """The inverse of split_observation (frames decoded in parallel)."""
    obs = decode_images(parts.get(IMAGES, {}))
    obs.update((k, decode_array(v)) for k, v in parts.get(ARRAYS, {}).items())
    obs.update(parts.get(STRINGS, {}))
    return obs


def encode_obs_fields(obs: dict, compress: bool = True):
    """(images, arrays, strings) payload dicts of an observation."""
    parts = split_observation(obs, compress)
    return tuple(parts[k] for k in KINDS)


def _obs_to_msgpack(parts: dict) -> bytes:
    wire = {}
    for kind in KINDS:
        tag = _ENVELOPE.get(kind)
        for key, payload in parts[kind].items():
            wire[key] = {tag: True, 'data': payload} if tag else payload
    return msgpack.packb(wire)


def _obs_from_msgpack(data: bytes) -> dict:
    """A msgpack observation map back to values, in its key order; values
    in no envelope pass through (bytes as UTF-8 text)."""
    found = {}    # key -> (kind or None, payload)
    for key, v in msgpack.unpackb(data, raw=False).items():
        kind = next((k for k, tag in _ENVELOPE.items()
                     if isinstance(v, dict) and tag in v), None)
        found[key] = (kind, v['data'] if kind else
                      (v.decode() if isinstance(v, bytes) else v))
    decoded = join_observation({k: {key: p for key, (kk, p) in found.items()
                                    if kk == k} for k in _ENVELOPE})
    return {key: decoded[key] if kind else p for key, (kind, p) in found.items()}


def _obs_to_proto(parts: dict):
    return _pb().Observation(**{k: parts[k] for k in KINDS})


def _obs_from_proto(msg) -> dict:
    return join_observation({k: dict(getattr(msg, k).items()) for k in KINDS})


# ---------------------------------------------------------------------------
# protobuf messages of vla_service.proto, built from a descriptor
# ---------------------------------------------------------------------------
_PB = None


def _pb():
    """Message classes (Observation, PredictActionRequest,
    PredictActionResponse) of package ``fluxvla``."""
    global _PB
    if _PB is not None:
        return _PB
    from google.protobuf import descriptor_pb2, descriptor_pool, message_factory
    F = descriptor_pb2.FieldDescriptorProto
    fd = descriptor_pb2.FileDescriptorProto(name='fluxvla_amd_vla_service.proto',
                                            package='fluxvla', syntax='proto3')

    def field(msg, name, num, ftype, label=F.LABEL_OPTIONAL, type_name=None):
        f = msg.field.add(name=name, number=num, type=ftype, label=label)
        if type_name:
            f.type_name = type_name

    obs = fd.message_type.add(name='Observation')
    for num, (name, vtype) in enumerate(((IMAGES, F.TYPE_BYTES),
                                         (ARRAYS, F.TYPE_BYTES),
                                         (STRINGS, F.TYPE_STRING)), 1):
        entry = name.capitalize() + 'Entry'
        e = obs.nested_type.add(name=entry)
        e.options.map_entry = True
        field(e, 'key', 1, F.TYPE_STRING)
        field(e, 'value', 2, vtype)
        field(obs, name, num, F.TYPE_MESSAGE, F.LABEL_REPEATED,
              f'.fluxvla.Observation.{entry}')
    req = fd.message_type.add(name='PredictActionRequest')
    field(req, 'obs', 1, F.TYPE_MESSAGE, type_name='.fluxvla.Observation')
    field(req, 'unnorm_key', 2, F.TYPE_STRING)
    resp = fd.message_type.add(name='PredictActionResponse')
    field(resp, 'action_data', 1, F.TYPE_BYTES)
    field(resp, 'infer_time', 2, F.TYPE_DOUBLE)
    field(resp, 'error', 3, F.TYPE_STRING)
    pool = descriptor_pool.DescriptorPool()
    pool.Add(fd)

    class PB:
        pass

    for name in ('Observation', 'PredictActionRequest', 'PredictActionResponse'):
        setattr(PB, name, message_factory.GetMessageClass(
            pool.FindMessageTypeByName(f'fluxvla.{name}')))
    _PB = PB
    return PB


def _tagged(message) -> bytes:
    return bytes([FORMAT_PROTOBUF]) + message.SerializeToString()


# ---------------------------------------------------------------------------
# requests and replies
# ---------------------------------------------------------------------------
def encode_predict_request(obs: dict, unnorm_key: str, fmt: str = 'msgpack',
                           compress: bool = True) -> bytes:
    """A predict_action request in ``fmt`` ('msgpack' or 'protobuf')."""
    parts = split_observation(obs, compress)
    if fmt == 'protobuf':
        return _tagged(_pb().PredictActionRequest(obs=_obs_to_proto(parts),
                                                  unnorm_key=unnorm_key))
    return msgpack.packb({'endpoint': 'predict_action',
                          'data': {'obs_data': _obs_to_msgpack(parts),
                                   'unnorm_key': unnorm_key}})


def decode_predict_request(raw: bytes) -> tuple[int, dict, str]:
    """-> (format tag, observation dict, unnorm_key)."""
    if detect_format(raw) == FORMAT_PROTOBUF:
        req = _pb().PredictActionRequest.FromString(raw[1:])
        return FORMAT_PROTOBUF, _obs_from_proto(req.obs), req.unnorm_key
    data = msgpack.unpackb(raw, raw=False).get('data', {})
    return (FORMAT_MSGPACK, _obs_from_msgpack(data['obs_data']),
            data.get('unnorm_key', ''))


def predict_reply(action_data: bytes, infer_time: float, error: str = '') -> dict:
    """The reply dict of predict_action: the error alone, or the actions
    and the inference time."""
    if error:
        return {'error': error}
    return {'action_data': action_data, 'infer_time': infer_time}


def encode_predict_response(action_data: bytes, infer_time: float,
                            fmt: int = FORMAT_MSGPACK, error: str = '') -> bytes:
    reply = predict_reply(action_data, infer_time, error)
    if fmt == FORMAT_PROTOBUF:
        return _tagged(_pb().PredictActionResponse(**reply))
    return msgpack.packb(reply)


def decode_predict_response(raw: bytes, fmt: int = FORMAT_MSGPACK) -> dict:
    if fmt != FORMAT_PROTOBUF:
        return msgpack.unpackb(raw, raw=False)
    resp = _pb().PredictActionResponse.FromString(raw[1:])
    return predict_reply(resp.action_data, resp.infer_time, resp.error)


# ---------------------------------------------------------------------------
# the reference's client-facing classes, over the functions above
# ---------------------------------------------------------------------------
def _tag_array(obj):
    if isinstance(obj, np.ndarray):
        return {'__ndarray__': True, 'data': encode_array(obj)}
    raise TypeError(f'Cannot serialize {type(obj)}')


def _untag_array(obj: dict):
    return decode_array(obj['data']) if '__ndarray__' in obj else obj


class MsgSerializer:
    """General msgpack payloads, numpy arrays inside as ``__ndarray__``
    maps (every map of the message is checked for the tag)."""

    @staticmethod
    def to_bytes(data: Any) -> bytes:
        return msgpack.packb(data, default=_tag_array)

    @staticmethod
    def from_bytes(data: bytes) -> Any:
        return msgpack.unpackb(data, object_hook=_untag_array)


class ObsSerializer:
    """Observation dicts as msgpack maps."""

    @staticmethod
    def to_bytes(obs: dict, compress: bool = True) -> bytes:
        return _obs_to_msgpack(split_observation(obs, compress))

    @staticmethod
    def from_bytes(data: bytes) -> dict:
        return _obs_from_msgpack(data)


class ObsSerializerProto:
    """Observation dicts as protobuf Observation messages."""

    @staticmethod
    def obs_to_proto(obs: dict, compress: bool = True):
        return _obs_to_proto(split_observation(obs, compress))

    @staticmethod
    def obs_from_proto(msg) -> dict:
        return _obs_from_proto(msg)
