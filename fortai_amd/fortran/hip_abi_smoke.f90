! hip_abi_smoke.f90 -- a Fortran caller of libfortai_hip.so through
! fortai_backend_hip, the way the reference model calls its device binding.
!
! Known answers are the reference's own (test/test_fortai_smoke.f90:213-265):
! one Q8_0 block with fp16 scale 1.0 and quants 1..32 (times 1, 2, 3) against
! an all-ones activation gives 527.9677734375, 1055.935546875 and
! 1583.9033203125 (the activation is Q8_0-quantized: scale fp16(1/127)).
! Exit status 0 and "fortran abi smoke ok" on success.
program hip_abi_smoke
    use, intrinsic :: iso_c_binding, only: c_float, c_int8_t, c_ptr, c_size_t, c_null_ptr
    use fortai_status, only: FORTAI_INVALID, status_t
    use fortai_backend_hip
    implicit none

    type(hip_q8_context_t) :: ctx
    type(hip_q8_weights_t) :: w1, w2, w3
    type(status_t) :: stat
    integer(c_int8_t), allocatable :: one(:), two(:), three(:), act(:)
    real(c_float) :: ones(32), dev_out(2), o1(1), o2(2), o3(1), ms
    type(c_ptr) :: x_dev, y_dev
    real(c_float), parameter :: a1 = 527.9677734375, a2 = 1055.935546875, a3 = 1583.9033203125
    integer :: failures

    failures = 0
    call ctx%create(0, stat)
    call need(stat%is_ok(), 'context create')
    one = q8_rows([1])
    two = q8_rows([1, 2])
    three = q8_rows([3])
    call w1%upload(ctx, one, int(size(one), c_size_t), 1, 32, stat)
    call need(stat%is_ok(), 'upload 1')
    call w2%upload(ctx, two, int(size(two), c_size_t), 2, 32, stat)
    call need(stat%is_ok(), 'upload 2')
    call w3%upload(ctx, three, int(size(three), c_size_t), 1, 32, stat)
    call need(stat%is_ok(), 'upload 3')

    ! device f32 activation, quantized on the device
    ones = 1.0_c_float
    call ctx%allocate_buffer(128_c_size_t, x_dev, stat)
    call need(stat%is_ok(), 'allocate x')
    call ctx%allocate_buffer(8_c_size_t, y_dev, stat)
    call need(stat%is_ok(), 'allocate y')
    call ctx%upload_real(x_dev, ones, stat)
    call need(stat%is_ok(), 'upload x')
    call hip_q8_matvec_device_f32(ctx, w2, x_dev, 32_c_size_t, y_dev, 2_c_size_t, stat)
    call need(stat%is_ok(), 'matvec_device_f32')
    call ctx%download_real(y_dev, dev_out, stat)
    call need(stat%is_ok(), 'download y')
    call need(dev_out(1) == a1 .and. dev_out(2) == a2, 'device matvec known answer')

    ! host Q8_0 activation: fp16(1/127) = 0x2008, quants 127
    allocate (act(34))
    act(1) = int(z'08', c_int8_t)
    act(2) = int(z'20', c_int8_t)
    act(3:) = 127_c_int8_t
    call hip_q8_matvec_host_triplet(ctx, w1, w2, w3, act, 34_c_size_t, o1, 4_c_size_t, o2, 8_c_size_t, &
        o3, 4_c_size_t, ms, stat)
    call need(stat%is_ok(), 'triplet')
    call need(o1(1) == a1 .and. o2(1) == a1 .and. o2(2) == a2 .and. o3(1) == a3, 'triplet known answer')

    ! argument checking happens before the C call
    call hip_q8_matvec_device_f32(ctx, w2, x_dev, 32_c_size_t, c_null_ptr, 2_c_size_t, stat)
    call need(stat%code == FORTAI_INVALID, 'null output is FORTAI_INVALID')

    call ctx%free_buffer(x_dev, stat)
    call ctx%free_buffer(y_dev, stat)
    call w1%destroy(stat)
    call w2%destroy(stat)
    call w3%destroy(stat)
    call ctx%destroy(stat)
    call need(stat%is_ok(), 'context destroy')
    if (failures /= 0) error stop 1
    print '(a)', 'fortran abi smoke ok'

contains

    ! rows of one Q8_0 block each: fp16 scale 1.0 (0x3c00), quants m*(1..32)
    function q8_rows(mult) result(bytes)
        integer, intent(in) :: mult(:)
        integer(c_int8_t), allocatable :: bytes(:)
        integer :: r, i
        allocate (bytes(34 * size(mult)))
        do r = 1, size(mult)
            bytes(34 * (r - 1) + 1) = 0_c_int8_t
            bytes(34 * (r - 1) + 2) = int(z'3c', c_int8_t)
            do i = 1, 32
                bytes(34 * (r - 1) + 2 + i) = int(mult(r) * i, c_int8_t)
            end do
        end do
    end function q8_rows

    subroutine need(ok, what)
        logical, intent(in) :: ok
        character(len=*), intent(in) :: what
        if (.not. ok) then
            failures = failures + 1
            print '(a)', 'FAILED: ' // what
            if (allocated(stat%message)) print '(a)', '  status: ' // stat%message
        end if
    end subroutine need

end program hip_abi_smoke
