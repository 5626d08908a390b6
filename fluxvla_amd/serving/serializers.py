"""Wire formats of the predict_action endpoint.

Byte-compatible with the reference's serializers
(fluxvla/engines/runners/serving/serializers.py:1-250) and its protobuf
schema (serving/proto/vla_service.proto), so a reference client talks to
this server unchanged:

* msgpack (default): ``{"endpoint": name, "data": {...}}``; an observation is
  a msgpack map whose values are ``{"__jpeg__": True, "data": jpeg}`` for
  compressed camera frames, ``{"__ndarray__": True, "data": npy}`` for
  arrays, or plain strings; responses carry the action tensor as .npy bytes.
* protobuf: first byte 0x01, then a PredictActionRequest /
  PredictActionResponse message.  The message classes are built at import
  from a descriptor equal to vla_service.proto (no generated code needed).

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

FORMAT_MSGPACK: int = 0x00
FORMAT_PROTOBUF: int = 0x01

JPEG_QUALITY = 95
JPEG_KEYS = frozenset({
    'cam_high', 'cam_left_wrist', 'cam_right_wrist', 'agentview_image',
    'robot0_eye_in_hand_image',
})


def detect_format(raw: bytes) -> int:
    """0x01 first byte: protobuf; anything else: msgpack."""
    return FORMAT_PROTOBUF if raw and raw[0] == FORMAT_PROTOBUF else FORMAT_MSGPACK


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
    buf = io.BytesIO()
    np.save(buf, arr, allow_pickle=False)
    return buf.getvalue()


def decode_array(data: bytes) -> np.ndarray:
    return np.load(io.BytesIO(data), allow_pickle=False)


def encode_obs_fields(obs: dict, compress: bool = True):
    """Observation -> (jpeg images, npy arrays, strings) dicts: uint8 HWC
    frames under the known camera keys are JPEG-compressed."""
    images, arrays, strings = {}, {}, {}
    for k, v in obs.items():
        if (compress and isinstance(v, np.ndarray) and v.ndim == 3
                and v.dtype == np.uint8 and k in JPEG_KEYS):
            images[k] = encode_image(v)
        elif isinstance(v, np.ndarray):
            arrays[k] = encode_array(v)
        elif isinstance(v, str):
            strings[k] = v
    return images, arrays, strings


class MsgSerializer:
    """msgpack with numpy arrays as ``{"__ndarray__": True, "data": npy}``."""

    @staticmethod
    def to_bytes(data: Any) -> bytes:
        return msgpack.packb(data, default=MsgSerializer._encode)

    @staticmethod
    def from_bytes(data: bytes) -> Any:
        return msgpack.unpackb(data, object_hook=MsgSerializer._decode)

    @staticmethod
    def _decode(obj):
        if '__ndarray__' in obj:
            return decode_array(obj['data'])
        return obj

    @staticmethod
    def _encode(obj):
        if isinstance(obj, np.ndarray):
            return {'__ndarray__': True, 'data': encode_array(obj)}
        raise TypeError(f'Cannot serialize {type(obj)}')


class ObsSerializer:
    """Observation dicts as msgpack maps."""

    @staticmethod
    def to_bytes(obs: dict, compress: bool = True) -> bytes:
        images, arrays, strings = encode_obs_fields(obs, compress)
        enc = {k: {'__jpeg__': True, 'data': v} for k, v in images.items()}
        enc.update({k: {'__ndarray__': True, 'data': v} for k, v in arrays.items()})
        enc.update(strings)
        return msgpack.packb(enc)

    @staticmethod
    def from_bytes(data: bytes) -> dict:
        obs, jpegs = {}, {}
        for k, v in msgpack.unpackb(data, raw=False).items():
            if isinstance(v, dict) and '__jpeg__' in v:
                jpegs[k] = v['data']
                obs[k] = None  # keeps the key order
            elif isinstance(v, dict) and '__ndarray__' in v:
                obs[k] = decode_array(v['data'])
            elif isinstance(v, bytes):
                obs[k] = v.decode()
            else:
                obs[k] = v
        obs.update(decode_images(jpegs))
        return obs


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
    for num, (name, vtype) in enumerate((('images', F.TYPE_BYTES),
                                         ('arrays', F.TYPE_BYTES),
                                         ('strings', F.TYPE_STRING)), 1):
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


class ObsSerializerProto:
    """Observation dicts as protobuf Observation messages."""

    @staticmethod
    def obs_to_proto(obs: dict, compress: bool = True):
        images, arrays, strings = encode_obs_fields(obs, compress)
        msg = _pb().Observation()
        for k, v in images.items():
            msg.images[k] = v
        for k, v in arrays.items():
            msg.arrays[k] = v
        for k, v in strings.items():
            msg.strings[k] = v
        return msg

    @staticmethod
    def obs_from_proto(msg) -> dict:
        obs = decode_images(dict(msg.images.items()))
        obs.update({k: decode_array(v) for k, v in msg.arrays.items()})
        obs.update(dict(msg.strings.items()))
        return obs


def encode_predict_request(obs: dict, unnorm_key: str, fmt: str = 'msgpack',
                           compress: bool = True) -> bytes:
    if fmt == 'protobuf':
        req = _pb().PredictActionRequest()
        req.obs.CopyFrom(ObsSerializerProto.obs_to_proto(obs, compress=compress))
        req.unnorm_key = unnorm_key
        return bytes([FORMAT_PROTOBUF]) + req.SerializeToString()
    return msgpack.packb({
        'endpoint': 'predict_action',
        'data': {'obs_data': ObsSerializer.to_bytes(obs, compress=compress),
                 'unnorm_key': unnorm_key},
    })


def decode_predict_request(raw: bytes) -> tuple[int, dict, str]:
    """-> (format tag, observation dict, unnorm_key)."""
    if detect_format(raw) == FORMAT_PROTOBUF:
        req = _pb().PredictActionRequest()
        req.ParseFromString(raw[1:])
        return FORMAT_PROTOBUF, ObsSerializerProto.obs_from_proto(req.obs), req.unnorm_key
    data = msgpack.unpackb(raw, raw=False).get('data', {})
    return (FORMAT_MSGPACK, ObsSerializer.from_bytes(data['obs_data']),
            data.get('unnorm_key', ''))


def encode_predict_response(action_data: bytes, infer_time: float,
                            fmt: int = FORMAT_MSGPACK, error: str = '') -> bytes:
    if fmt == FORMAT_PROTOBUF:
        resp = _pb().PredictActionResponse()
        if error:
            resp.error = error
        else:
            resp.action_data = action_data
            resp.infer_time = infer_time
        return bytes([FORMAT_PROTOBUF]) + resp.SerializeToString()
    if error:
        return msgpack.packb({'error': error})
    return msgpack.packb({'action_data': action_data, 'infer_time': infer_time})


def decode_predict_response(raw: bytes, fmt: int = FORMAT_MSGPACK) -> dict:
    if fmt == FORMAT_PROTOBUF:
        resp = _pb().PredictActionResponse()
        resp.ParseFromString(raw[1:])
        if resp.error:
            return {'error': resp.error}
        return {'action_data': resp.action_data, 'infer_time': resp.infer_time}
    return msgpack.unpackb(raw, raw=False)
