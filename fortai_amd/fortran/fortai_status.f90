! fortai_status.f90 -- status object for standalone builds of the HIP binding.
!
! Inside the reference tree the reference's own src/fortai_status.f90 is used
! instead; this module keeps the same public names (src/fortai_status.f90:6-19:
! the FORTAI_* codes and status_t with code, message, clear, is_ok, set) so
! fortai_backend_hip.f90 compiles against either.
module fortai_status
    use, intrinsic :: iso_fortran_env, only: int32
    implicit none
    private

    integer(int32), parameter, public :: FORTAI_OK = 0_int32
    integer(int32), parameter, public :: FORTAI_INVALID = 1_int32
    integer(int32), parameter, public :: FORTAI_UNSUPPORTED = 2_int32
    integer(int32), parameter, public :: FORTAI_IO_ERROR = 3_int32
    integer(int32), parameter, public :: FORTAI_OUT_OF_MEMORY = 4_int32

    type, public :: status_t
        integer(int32) :: code = FORTAI_OK
        character(len=:), allocatable :: message
    contains
        procedure :: clear
        procedure :: is_ok
        procedure :: set
    end type status_t

contains

    subroutine clear(self)
        class(status_t), intent(inout) :: self
        self%code = FORTAI_OK
        if (allocated(self%message)) deallocate (self%message)
    end subroutine clear

    logical function is_ok(self)
        class(status_t), intent(in) :: self
        is_ok = self%code == FORTAI_OK
    end function is_ok

    subroutine set(self, code, message)
        class(status_t), intent(inout) :: self
        integer(int32), intent(in) :: code
        character(len=*), intent(in), optional :: message
        self%code = code
        if (present(message)) then
            self%message = message
        else if (allocated(self%message)) then
            deallocate (self%message)
        end if
    end subroutine set

end module fortai_status
