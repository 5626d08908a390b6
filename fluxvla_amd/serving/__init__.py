"""Serving boundary of the action-chunk path: the reference's predict_action
endpoint and wire formats (fluxvla/engines/runners/serving/), over the HIP
inference model."""
from .serializers import (FORMAT_MSGPACK, FORMAT_PROTOBUF, MsgSerializer,  # noqa: F401
                          ObsSerializer, ObsSerializerProto,
                          decode_predict_request, decode_predict_response,
                          detect_format, encode_predict_request,
                          encode_predict_response)
from .server import (ChunkEndpoint, ObsToInputs, PolicyServer,  # noqa: F401
                     create_server)
