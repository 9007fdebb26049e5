from ferrite.profiling.report import compile_report
from ferrite.profiling.roofline import KernelRoofline, RooflinePoint, analyze, format_table, traffic_bytes
from ferrite.profiling.timing import Timing, timeit
from ferrite.profiling.trace import trace

__all__ = ["compile_report", "KernelRoofline", "RooflinePoint", "analyze", "format_table", "traffic_bytes", "Timing", "timeit", "trace"]
