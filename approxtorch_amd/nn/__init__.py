from .Conv2d_int8 import Conv2d_int8
from .Conv2d_uint8 import Conv2d_uint8, uint8_qparams
from . import bgemm_int8
from . import bgemm_uint8
from . import quantization
