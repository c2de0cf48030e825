! fortai_backend_cuda_on_hip.f90 -- drop-in replacement for the reference's
! src/backend/cuda/fortai_backend_cuda.f90.
!
! It provides module fortai_backend_cuda with every public name the reference
! model code imports (src/models/qwen35/fortai_qwen35_cpu.f90:5-10,
! src/fortai.f90:4-5), each one the HIP implementation from
! fortai_backend_hip under its cuda_* name.  Building the reference with this
! file in place of its own binding (and linking libfortai_hip.so instead of
! the CUDA library) runs the reference's device pipeline on gfx950 with no
! change to the model sources.
module fortai_backend_cuda
    use, intrinsic :: iso_c_binding, only: c_int
    use fortai_backend_hip, only: &
        cuda_q8_context_t => hip_q8_context_t, &
        cuda_q8_weights_t => hip_q8_weights_t, &
        cuda_qwen35_recurrent_t => hip_qwen35_recurrent_t, &
        cuda_qwen35_attention_t => hip_qwen35_attention_t, &
        cuda_q8_matvec_host => hip_q8_matvec_host, &
        cuda_q8_matvec_host_pair => hip_q8_matvec_host_pair, &
        cuda_q8_matvec_host_triplet => hip_q8_matvec_host_triplet, &
        cuda_q8_matvec_host_triplet_contiguous => hip_q8_matvec_host_triplet_contiguous, &
        cuda_q8_ffn_host => hip_q8_ffn_host, &
        cuda_q8_ffn_device => hip_q8_ffn_device, &
        cuda_qwen35_copy_device => hip_qwen35_copy_device, &
        cuda_qwen35_add_device => hip_qwen35_add_device, &
        cuda_qwen35_rms_norm_device => hip_qwen35_rms_norm_device, &
        cuda_q8_matvec_resident => hip_q8_matvec_resident, &
        cuda_q8_matvec_device_f32 => hip_q8_matvec_device_f32, &
        cuda_qwen35_embedding_device => hip_qwen35_embedding_device
    implicit none
    private

    integer(c_int), parameter, public :: FORTAI_CUDA_OK = 0_c_int
    public :: cuda_q8_context_t, cuda_q8_weights_t, cuda_qwen35_recurrent_t, cuda_qwen35_attention_t
    public :: cuda_q8_matvec_host, cuda_q8_matvec_host_pair, cuda_q8_matvec_host_triplet
    public :: cuda_q8_matvec_host_triplet_contiguous, cuda_q8_ffn_host, cuda_q8_ffn_device
    public :: cuda_qwen35_copy_device, cuda_qwen35_add_device, cuda_qwen35_rms_norm_device
    public :: cuda_q8_matvec_resident, cuda_q8_matvec_device_f32, cuda_qwen35_embedding_device
end module fortai_backend_cuda
