! fortai_hip_plan.f90 -- the HIP decoders' execution plans as the reference's
! PlanIR.
!
! FortAI records an execution plan as plan_ir_t, one plan_step_t (operation,
! kernel, batch size) per step (src/fortai_plan_ir.f90:7-21).  The HIP
! decoders note every kernel a decode step launches when the step is
! captured: fortai_hip_qwen35_decoder_plan / _batch_plan return them as text,
! one "operation<TAB>kernel<TAB>batch" line per launch.  These procedures turn
! that text into plan_ir_t steps through plan_ir_t%append, in launch order,
! and end with plan_ir_t%validate.  The module is compiled against the
! reference's fortai_plan_ir and fortai_status.
module fortai_hip_plan
    use, intrinsic :: iso_fortran_env, only: int32
    use fortai_status, only: FORTAI_INVALID, status_t
    use fortai_plan_ir, only: plan_ir_t
    use fortai_backend_hip, only: hip_qwen35_decoder_t, hip_qwen35_batch_t
    implicit none
    private

    public :: hip_decoder_plan_ir, hip_batch_plan_ir, hip_plan_text_to_ir

contains

    ! plan := the launches of one decode step of the fused decoder
    subroutine hip_decoder_plan_ir(decoder, plan, stat)
        type(hip_qwen35_decoder_t), intent(in) :: decoder
        type(plan_ir_t), intent(inout) :: plan
        type(status_t), intent(out) :: stat
        character(len=:), allocatable :: text

        call decoder%plan(text, stat)
        if (.not. stat%is_ok()) return
        call hip_plan_text_to_ir(text, plan, stat)
    end subroutine hip_decoder_plan_ir

    ! plan := the launches of one batched step (prefill false) or of the
    ! last prompt prefill (prefill true); batch sizes as launched
    subroutine hip_batch_plan_ir(batch, prefill, plan, stat)
        type(hip_qwen35_batch_t), intent(in) :: batch
        logical, intent(in) :: prefill
        type(plan_ir_t), intent(inout) :: plan
        type(status_t), intent(out) :: stat
        character(len=:), allocatable :: text

        call batch%plan(prefill, text, stat)
        if (.not. stat%is_ok()) return
        call hip_plan_text_to_ir(text, plan, stat)
    end subroutine hip_batch_plan_ir

    ! plan := one step per line of text ("operation<TAB>kernel<TAB>batch",
    ! lines separated by LF); plan is cleared first and validated last
    subroutine hip_plan_text_to_ir(text, plan, stat)
        character(len=*), intent(in) :: text
        type(plan_ir_t), intent(inout) :: plan
        type(status_t), intent(out) :: stat
        character(len=1), parameter :: tab = achar(9), lf = achar(10)
        integer :: first, last, t1, t2, ios
        integer(int32) :: batch

        call stat%clear()
        call plan%clear()
        first = 1
        do while (first <= len(text))
            last = index(text(first:), lf)
            if (last == 0) then
                last = len(text)
            else
                last = first + last - 2
            end if
            if (last >= first) then
                t1 = index(text(first:last), tab)
                t2 = 0
                if (t1 > 0) t2 = index(text(first + t1:last), tab)
                if (t1 <= 1 .or. t2 <= 1) then
                    call stat%set(FORTAI_INVALID, 'HIP plan line without operation, kernel and batch: ' // &
                        text(first:last))
                    return
                end if
                t1 = first + t1 - 1          ! first tab
                t2 = t1 + t2                 ! second tab
                read (text(t2 + 1:last), *, iostat=ios) batch
                if (ios /= 0) then
                    call stat%set(FORTAI_INVALID, 'HIP plan line with a bad batch size: ' // text(first:last))
                    return
                end if
                call plan%append(text(first:t1 - 1), text(t1 + 1:t2 - 1), batch, stat)
                if (.not. stat%is_ok()) return
            end if
            first = last + 2
        end do
        call plan%validate(stat)
    end subroutine hip_plan_text_to_ir

end module fortai_hip_plan
