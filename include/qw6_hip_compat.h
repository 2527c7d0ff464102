/* qw6_hip_compat.h -- qw6's Vulkan host-op names on top of qw6_hip.h.
 *
 * A qw6 build with -DQW6_HIP includes this header where it includes
 * qw6_vk.h: every host operation of the MoE path that qw6_vk.h declares
 * (qw6_vk.h:9-56) then resolves to the HIP library's function with the same
 * parameter list and the same 0 / -1 return convention, so the call sites
 * of those host ops (qw6.c's GPU probes, qw6.c:1877, 1926, and
 * `qw6 --vulkan-self-test`, qw6.c:3540) relink unchanged.
 *
 * Not covered: the device-resident pipeline of qw6_vk.h:60-83
 * (qw6_vk_pipe_t, qw6_vk_pipe_init, qw6_vk_pipe_forward,
 * qw6_vk_pipe_forward_greedy, qw6_vk_pipe_free), which qw6.c's QW6_VULKAN
 * blocks call (qw6.c:2436-2441, 3696, 3714, 3887); a build with those blocks on
 * does not compile against this header alone. Their MoE-path roles have
 * HIP entry points with other signatures: qw6_hip_ctx_init / _free (the
 * pipe's lifetime), qw6_hip_upload and qw6_hip_experts_create (its weight
 * upload), qw6_hip_moe_forward (the MoE section of its forward) and
 * qw6_hip_output_greedy (its greedy head). Host ops of qw6_vk.h outside the
 * MoE FFN path (attention, DeltaNet, M-RoPE, the MTP draft head, the
 * per-group RMSNorm) have no HIP counterpart here; a build that needs them
 * keeps qw6's CPU path for them.
 */
#ifndef QW6_HIP_COMPAT_H
#define QW6_HIP_COMPAT_H

#include "qw6_hip.h"

#define qw6_vk_selftest             qw6_hip_selftest
#define qw6_vk_matvec_f32_host      qw6_hip_matvec_f32_host
#define qw6_vk_matmul_q4k_host      qw6_hip_matmul_q4k_host
#define qw6_vk_matmul_q5k_host      qw6_hip_matmul_q5k_host
#define qw6_vk_matmul_q6k_host      qw6_hip_matmul_q6k_host
#define qw6_vk_matmul_iq2xxs_host   qw6_hip_matmul_iq2xxs_host
#define qw6_vk_rmsnorm_host         qw6_hip_rmsnorm_host
#define qw6_vk_silu_mul_host        qw6_hip_silu_mul_host
#define qw6_vk_argmax_host          qw6_hip_argmax_host
#define qw6_vk_sampling_greedy_host qw6_hip_sampling_greedy_host
#define qw6_vk_moe_route_host       qw6_hip_moe_route_host
#define qw6_vk_moe_gather_host      qw6_hip_moe_gather_host

#endif
