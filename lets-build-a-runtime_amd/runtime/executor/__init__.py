from .common import Executor, COpNode, MAX_DIMS, MAX_INPUTS, OpTiming, RunProfile  # noqa: F401
from .compiled import CompiledExecutor, DeviceWeights  # noqa: F401
from .hip_lib import HipExecutorError, load_library  # noqa: F401
