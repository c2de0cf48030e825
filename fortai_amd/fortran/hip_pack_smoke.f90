! hip_pack_smoke.f90 -- a Fortran caller of the pack cache (fortai_hip_pack_cache).
!
! usage: hip_pack_smoke GGUF ROOT write|read
!
! Both modes upload three Q8_0 matrices of a fixed pseudo-random content the
! ordinary way (fortai_hip_q8_weights_upload, repacked on the device) and take
! their matvecs of a fixed activation.  write: pack them into
! hip_pack_path(ROOT, 'packsmoke') keyed by the GGUF's digest.  Both modes then
! open that pack, upload every matrix from it (no repack) and require the
! matvecs to equal the unpacked ones bit for bit; a stale digest and a wrong
! shape must be refused.  The reference's own key check
! (test/test_fortai_smoke.f90:182-194) runs first.
! Prints "pack <path>" and, on success, "fortran pack cache ok".
program hip_pack_smoke
    use, intrinsic :: iso_c_binding, only: c_float, c_int8_t, c_int32_t, c_ptr, c_size_t
    use fortai_status, only: FORTAI_INVALID, FORTAI_UNSUPPORTED, status_t
    use fortai_cache, only: pack_key_t, cache_path
    use fortai_backend_hip
    use fortai_hip_pack_cache
    implicit none

    integer, parameter :: n = 3
    integer, parameter :: rows(n) = [13, 200, 64], widths(n) = [96, 1024, 256]
    character(len=8), parameter :: names(n) = ['blk.0.a ', 'blk.0.bb', 'output  ']
    character(len=:), allocatable :: gguf, root, mode, path
    type(pack_key_t) :: key
    type(hip_q8_context_t) :: ctx
    type(hip_q8_weights_t) :: fresh(n), packed(n), spare
    type(hip_pack_writer_t) :: writer
    type(hip_pack_reader_t) :: reader
    type(status_t) :: stat
    integer(c_int8_t) :: digest(32), other(32)
    integer(c_int8_t), allocatable :: bytes(:)
    real(c_float), allocatable :: act(:), want(:, :), got(:)
    type(c_ptr) :: x_dev, y_dev
    integer :: failures, i
    integer(8) :: seed

    failures = 0
    gguf = argument(1)
    root = argument(2)
    mode = argument(3)

    ! the reference's key check, then this backend's key through the same rule
    key%model = 'qwen35'
    key%backend = 'cuda'
    key%variant = 'sm86'
    call need(cache_path('/tmp/fortai', key) == '/tmp/fortai/qwen35/cuda-sm86-abi1.pack', 'reference cache_path')
    call need(hip_pack_path('/tmp/fortai', 'qwen35') == '/tmp/fortai/qwen35/hip-gfx950-q8-lanes-abi1.pack', &
        'hip pack path')
    call need(hip_pack_path('/tmp/fortai', '') == '/tmp/fortai/invalid.pack', 'invalid key path')
    path = hip_pack_path(root, 'packsmoke')
    print '(a)', 'pack ' // path

    call hip_gguf_digest(gguf, digest, stat)
    call need(stat%is_ok(), 'gguf digest')
    call ctx%create(0, stat)
    call need(stat%is_ok(), 'context create')
    if (failures /= 0) error stop 1

    ! unpacked uploads and their matvecs
    allocate (act(maxval(widths)), want(maxval(rows), n), got(maxval(rows)))
    seed = 12345
    do i = 1, size(act)
        act(i) = real(next(seed), c_float) / 2147483648.0 - 0.5
    end do
    call ctx%allocate_buffer(int(4 * size(act), c_size_t), x_dev, stat)
    call ctx%allocate_buffer(int(4 * size(got), c_size_t), y_dev, stat)
    call ctx%upload_real(x_dev, act, stat)
    do i = 1, n
        bytes = q8_matrix(rows(i), widths(i), int(i, 8))
        call fresh(i)%upload(ctx, bytes, int(size(bytes), c_size_t), rows(i), widths(i), stat)
        call need(stat%is_ok(), 'upload ' // trim(names(i)))
        want(1:rows(i), i) = matvec(fresh(i), rows(i), widths(i))
    end do

    if (mode == 'write') then
        call writer%open(path, digest, stat)
        call need(stat%is_ok(), 'writer open')
        do i = 1, n
            call writer%add(trim(names(i)), fresh(i), rows(i), widths(i), stat)
            call need(stat%is_ok(), 'writer add ' // trim(names(i)))
        end do
        call writer%close(stat)
        call need(stat%is_ok(), 'writer close')
    end if

    ! a stale digest is refused, the right one opens
    other = digest
    other(1) = int(ieor(int(other(1)), 1), c_int8_t)
    call reader%open(path, other, stat)
    call need(stat%code == FORTAI_UNSUPPORTED, 'stale pack refused')
    call reader%open(path, digest, stat)
    call need(stat%is_ok(), 'reader open')
    if (failures /= 0) error stop 1
    do i = 1, n
        call reader%upload(trim(names(i)), ctx, packed(i), rows(i), widths(i), stat)
        call need(stat%is_ok(), 'packed upload ' // trim(names(i)))
        got(1:rows(i)) = matvec(packed(i), rows(i), widths(i))
        call need(all(transfer(got(1:rows(i)), 0_c_int32_t, rows(i)) == &
            transfer(want(1:rows(i), i), 0_c_int32_t, rows(i))), 'packed matvec bits ' // trim(names(i)))
    end do
    call reader%upload('blk.0.a', ctx, spare, rows(1) + 1, widths(1), stat)
    call need(stat%code == FORTAI_INVALID, 'wrong shape refused')
    call reader%upload('absent', ctx, spare, rows(1), widths(1), stat)
    call need(stat%code == FORTAI_INVALID, 'absent record refused')
    call reader%close()

    do i = 1, n
        call fresh(i)%destroy(stat)
        call packed(i)%destroy(stat)
    end do
    call ctx%free_buffer(x_dev, stat)
    call ctx%free_buffer(y_dev, stat)
    call ctx%destroy(stat)
    if (failures /= 0) error stop 1
    print '(a)', 'fortran pack cache ok'

contains

    function argument(i) result(text)
        integer, intent(in) :: i
        character(len=:), allocatable :: text
        integer :: length
        call get_command_argument(i, length=length)
        allocate (character(len=length) :: text)
        if (length > 0) call get_command_argument(i, text)
    end function argument

    ! 31-bit linear congruential stream
    integer function next(s)
        integer(8), intent(inout) :: s
        s = modulo(s * 1103515245_8 + 12345_8, 2147483648_8)
        next = int(s)
    end function next

    ! GGUF Q8_0 bytes: per block an fp16 scale in [2^-10, 2^-6) and 32 quants
    function q8_matrix(r, w, salt) result(b)
        integer, intent(in) :: r, w
        integer(8), intent(in) :: salt
        integer(c_int8_t), allocatable :: b(:)
        integer(8) :: s
        integer :: blk, j, v, base
        allocate (b(r * (w / 32) * 34))
        s = salt * 7919_8
        do blk = 0, r * (w / 32) - 1
            base = blk * 34
            v = 5120 + modulo(next(s), 4096)  ! fp16 bits 0x1400..0x23ff
            b(base + 1) = int(iand(v, 255) - merge(256, 0, iand(v, 255) > 127), c_int8_t)
            b(base + 2) = int(ishft(v, -8), c_int8_t)
            do j = 1, 32
                b(base + 2 + j) = int(modulo(next(s), 255) - 127, c_int8_t)
            end do
        end do
    end function q8_matrix

    function matvec(weights, r, w) result(y)
        type(hip_q8_weights_t), intent(in) :: weights
        integer, intent(in) :: r, w
        real(c_float) :: y(r)
        real(c_float) :: buffer(maxval(rows))
        call hip_q8_matvec_device_f32(ctx, weights, x_dev, int(w, c_size_t), y_dev, int(r, c_size_t), stat)
        call need(stat%is_ok(), 'matvec')
        call ctx%download_real(y_dev, buffer, stat)
        y = buffer(1:r)
    end function matvec

    subroutine need(ok, what)
        logical, intent(in) :: ok
        character(len=*), intent(in) :: what
        if (.not. ok) then
            failures = failures + 1
            print '(a)', 'FAILED: ' // what
            if (allocated(stat%message)) print '(a)', '  status: ' // stat%message
        end if
    end subroutine need

end program hip_pack_smoke
