"""Host-side problem definitions producing batched QP blocks."""
from .ocp import LinearOCP, QuadraticTrackingOCP  # noqa: F401
from .quadrotor import QuadrotorOCP, QUAD_PARAMS  # noqa: F401
