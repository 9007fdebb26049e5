from ferrite.profiling.report import compile_report
from ferrite.profiling.roofline import RooflinePoint, analyze, format_table
from ferrite.profiling.timing import Timing, timeit
from ferrite.profiling.trace import trace

__all__ = ["compile_report", "RooflinePoint", "analyze", "format_table", "Timing", "timeit", "trace"]
