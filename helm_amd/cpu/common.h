// Internal helpers shared by the sources of libhelm_cpu.so (not exported).
#ifndef HELM_CPU_COMMON_H
#define HELM_CPU_COMMON_H

#include <string>

namespace helm_cpu_internal {

// Records `msg` as this thread's last error (helm_cpu_last_error) and returns code.
int fail(int code, const std::string& msg);
const char* last_error();
// HELM_CPU_ISA_*: AVX-512 (F + BW + VL) when the CPU has it, else AVX2 + F16C +
// FMA, else none; environment HELM_CPU_ISA=avx2 caps it at AVX2.
int detect_isa();

}  // namespace helm_cpu_internal

#endif  // HELM_CPU_COMMON_H
